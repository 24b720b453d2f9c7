// Fused pair transition: out = [x +] mask * W_o( silu(W_a n) * (W_b n) ), n = LayerNorm(x).
// Replaces common/opt_core/opt_core/kernels/transition/__init__.py:1074 (transition) / attn/pair_fused.py:1519.
//
// bf16 path (c = 128): one wave owns PW x 32 pixel rows.  LN runs in registers and leaves the normalised rows as the
// B operand of v_mfma_f32_32x32x16_bf16 (lane n%32 = pixel, channels 64*(lane/32) + 8t .. +7 for k-step t).  GEMM 1 is
// computed transposed, a^T = W_a n^T, so its D layout (lane = pixel, 16 hidden values) IS the B operand of GEMM 2
// out^T = W_o h^T once the hidden index of each k-step is permuted the same way in W_o: the 4c hidden never leaves the
// registers.  Weights stream through double-buffered LDS in 32-hidden chunks shared by the 8 waves of a workgroup (the next
// chunk's global loads are in flight while the current one feeds the MFMAs; one barrier per chunk).
// fp32 path (exact tier): LDS-tiled scalar FMA, fp32 throughout.
#include "rowtile.h"

namespace fpf {

constexpr int TR_C = 128;
constexpr int TR_KS = TR_C / 16;      // k-steps of GEMM 1
constexpr int TR_HB = 32;             // hidden rows per chunk
constexpr int TR_WLD = TR_C + 8;      // LDS pitch of a W_a / W_b chunk row (bf16): 272 B, conflict-free 16-byte reads
constexpr int TR_OLD = TR_HB + 4;     // LDS pitch of a W_o chunk row (bf16): 72 B, conflict-free 8-byte reads
constexpr int TR_WAVES = 8;           // waves per workgroup (2 per SIMD), 32 pixel rows each

template <int PW>
__global__ void __launch_bounds__(512) transition_bf16_kernel(const uint16_t* x, uint16_t* out, const float* __restrict__ ln_w,
                                                              const float* __restrict__ ln_b, float eps, const uint16_t* __restrict__ wa,
                                                              const uint16_t* __restrict__ wb, const uint16_t* __restrict__ wo,
                                                              const float* __restrict__ mask, int residual, int64_t rows, int hidden) {
  // double-buffered weight chunks: W_a / W_b rows hb*32 .. +31 (all 128 inputs) and W_o columns hb*32 .. +31 (all 128 outputs)
  __shared__ __attribute__((aligned(16))) uint16_t sWa[2][TR_HB * TR_WLD];
  __shared__ __attribute__((aligned(16))) uint16_t sWb[2][TR_HB * TR_WLD];
  __shared__ __attribute__((aligned(16))) uint16_t sWo[2][TR_C * TR_OLD];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, n = l & 31, g = l >> 5;
  const int64_t pix0 = ((int64_t)blockIdx.x * TR_WAVES + wave) * (32 * PW);
  // staging map: 1536 16-byte chunks per weight chunk (512 W_a, 512 W_b, 512 W_o), 3 per thread
  const int sr = tid >> 4, sc = tid & 15;          // W_a / W_b: row, 16-byte column
  const int so = tid >> 2, soc = tid & 3;          // W_o: row (c_out), 16-byte column within the 32 hidden
  u32x4 pa, pb, po;
  auto gload = [&](int hb) {
    pa = *reinterpret_cast<const u32x4*>(wa + (int64_t)(hb * TR_HB + sr) * TR_C + sc * 8);
    pb = *reinterpret_cast<const u32x4*>(wb + (int64_t)(hb * TR_HB + sr) * TR_C + sc * 8);
    po = *reinterpret_cast<const u32x4*>(wo + (int64_t)so * hidden + hb * TR_HB + soc * 8);
  };
  auto lstore = [&](int buf) {
    *reinterpret_cast<u32x4*>(&sWa[buf][sr * TR_WLD + sc * 8]) = pa;
    *reinterpret_cast<u32x4*>(&sWb[buf][sr * TR_WLD + sc * 8]) = pb;
    *reinterpret_cast<u32x2*>(&sWo[buf][so * TR_OLD + soc * 8]) = u32x2{po[0], po[1]};
    *reinterpret_cast<u32x2*>(&sWo[buf][so * TR_OLD + soc * 8 + 4]) = u32x2{po[2], po[3]};
  };
  __shared__ __attribute__((aligned(16))) float sLN[2 * RT_C];
  rt_stage_affine(sLN, ln_w, ln_b, tid, 512);
  gload(0);
  lstore(0);
  __syncthreads();
  bf16x8 xb[PW][TR_KS];
#pragma unroll
  for (int p = 0; p < PW; ++p) {
    const int64_t pix = pix0 + 32 * p + n;
    u32x4 raw[8];
    rt_load(x + (pix < rows ? pix : 0) * TR_C, pix < rows, g, raw);
    rt_ln(raw, g, sLN, eps, xb[p]);
  }
  f32x16 acc[PW][4];
#pragma unroll
  for (int p = 0; p < PW; ++p)
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) acc[p][cb] = f32x16{};
  const int nhb = hidden / TR_HB;
  for (int hb = 0; hb < nhb; ++hb) {
    const int buf = hb & 1;
    if (hb + 1 < nhb) gload(hb + 1);
    f32x16 a[PW], b[PW];
#pragma unroll
    for (int p = 0; p < PW; ++p) {
      a[p] = f32x16{};
      b[p] = f32x16{};
    }
    const uint16_t* ra = &sWa[buf][n * TR_WLD + 64 * g];
    const uint16_t* rb = &sWb[buf][n * TR_WLD + 64 * g];
    bf16x8 fa = as_bf8(*reinterpret_cast<const u32x4*>(ra)), fb = as_bf8(*reinterpret_cast<const u32x4*>(rb));
#pragma unroll
    for (int t = 0; t < TR_KS; ++t) {
      const bf16x8 ca = fa, cbf = fb;
      if (t + 1 < TR_KS) {                      // one k-step of fragment lookahead
        fa = as_bf8(*reinterpret_cast<const u32x4*>(ra + 8 * (t + 1)));
        fb = as_bf8(*reinterpret_cast<const u32x4*>(rb + 8 * (t + 1)));
      }
#pragma unroll
      for (int p = 0; p < PW; ++p) {
        a[p] = mfma32(ca, xb[p][t], a[p]);
        b[p] = mfma32(cbf, xb[p][t], b[p]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // h = silu(a) * b; registers 8s .. 8s+7 form the B operand of k-step s (hidden 16s + 8(e/4) + 4g + e%4)
    bf16x8 hf[PW][2];
#pragma unroll
    for (int p = 0; p < PW; ++p)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int v0 = 8 * s + 2 * e;
          const float a0 = a[p][v0], a1 = a[p][v0 + 1];
          const float h0 = siluf_(a0) * b[p][v0];
          const float h1 = siluf_(a1) * b[p][v0 + 1];
          w[e] = pack2(h0, h1);
        }
        hf[p][s] = as_bf8(u32x4{w[0], w[1], w[2], w[3]});
      }
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const uint16_t* wrow = &sWo[buf][(cb * 32 + n) * TR_OLD + 16 * s + 4 * g];
        const u32x2 lo = *reinterpret_cast<const u32x2*>(wrow);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(wrow + 8);
        const bf16x8 fo = as_bf8(u32x4{lo[0], lo[1], hi[0], hi[1]});
#pragma unroll
        for (int p = 0; p < PW; ++p) acc[p][cb] = mfma32(fo, hf[p][s], acc[p][cb]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (hb + 1 < nhb) lstore(buf ^ 1);        // buf ^ 1 was last read before the previous barrier
    __syncthreads();
  }
  // epilogue: lane (pixel n, half g) holds c_out = 32 cb + c_row(v, g); after the lane exchange it holds channels
  // 32 cb + 8g .. +7 and 32 cb + 16 + 8g .. +7, stored (with mask and residual) in 16-byte pieces
#pragma unroll
  for (int p = 0; p < PW; ++p) {
    const int64_t pix = pix0 + 32 * p + n;
    const bool live = pix < rows;
    const float m = (mask && live) ? mask[pix] : 1.0f;
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      float y[16];
      rt_regroup_f32(acc[p][cb], y);
      if (!live) continue;
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const int64_t c0 = pix * TR_C + 32 * cb + 16 * h2 + 8 * g;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = y[8 * h2 + e] * m;
        if (residual) {
          const u32x4 r = *reinterpret_cast<const u32x4*>(x + c0);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[2 * e] += lo_bf(r[e]);
            v[2 * e + 1] += hi_bf(r[e]);
          }
        }
        *reinterpret_cast<u32x4*>(out + c0) = u32x4{pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7])};
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------- fp32 (exact tier)
constexpr int TF_R = 32;    // rows per workgroup
constexpr int TF_HC = 16;   // hidden per chunk
constexpr int TF_CM = 128;  // max c

__global__ void __launch_bounds__(256) transition_f32_kernel(const float* x, float* out, const float* __restrict__ ln_w,
                                                             const float* __restrict__ ln_b, float eps, const float* __restrict__ wa,
                                                             const float* __restrict__ wb, const float* __restrict__ wo,
                                                             const float* __restrict__ mask, int residual, int64_t rows, int c, int hidden) {
  __shared__ float xs[TF_R][TF_CM + 1];
  __shared__ float was[TF_HC][TF_CM + 1];
  __shared__ float wbs[TF_HC][TF_CM + 1];
  __shared__ float wos[TF_CM][TF_HC + 1];
  __shared__ float hs[TF_R][TF_HC + 1];
  const int tid = threadIdx.x;
  const int r = tid >> 3, sub = tid & 7;   // 8 threads per row
  const int64_t row0 = (int64_t)blockIdx.x * TF_R;
  const int64_t row = row0 + r;
  const bool live = row < rows;
  // LayerNorm: 8 threads per row, strided channels
  float s = 0.f;
  for (int cc = sub; cc < c; cc += 8) s += live ? x[row * c + cc] : 0.f;
  for (int o = 4; o >= 1; o >>= 1) s += __shfl_xor(s, o, 8);
  const float mean = s / (float)c;
  float q = 0.f;
  for (int cc = sub; cc < c; cc += 8) {
    const float d = (live ? x[row * c + cc] : 0.f) - mean;
    q += d * d;
  }
  for (int o = 4; o >= 1; o >>= 1) q += __shfl_xor(q, o, 8);
  const float rstd = 1.0f / sqrtf(q / (float)c + eps);
  for (int cc = sub; cc < c; cc += 8) {
    const float v = live ? x[row * c + cc] : 0.f;
    xs[r][cc] = (v - mean) * rstd * (ln_w ? ln_w[cc] : 1.f) + (ln_b ? ln_b[cc] : 0.f);
  }
  float acc[TF_CM / 8];
#pragma unroll
  for (int i = 0; i < TF_CM / 8; ++i) acc[i] = 0.f;
  for (int h0 = 0; h0 < hidden; h0 += TF_HC) {
    const int hc = min(TF_HC, hidden - h0);
    __syncthreads();
    for (int i = tid; i < TF_HC * c; i += 256) {
      const int j = i / c, cc = i % c;
      was[j][cc] = j < hc ? wa[(int64_t)(h0 + j) * c + cc] : 0.f;
      wbs[j][cc] = j < hc ? wb[(int64_t)(h0 + j) * c + cc] : 0.f;
    }
    for (int i = tid; i < c * TF_HC; i += 256) {
      const int cc = i / TF_HC, j = i % TF_HC;
      wos[cc][j] = j < hc ? wo[(int64_t)cc * hidden + h0 + j] : 0.f;
    }
    __syncthreads();
    for (int jj = 0; jj < 2; ++jj) {
      const int j = sub * 2 + jj;
      float av = 0.f, bv = 0.f;
      for (int cc = 0; cc < c; ++cc) {
        av = fmaf(xs[r][cc], was[j][cc], av);
        bv = fmaf(xs[r][cc], wbs[j][cc], bv);
      }
      hs[r][j] = av / (1.0f + expf(-av)) * bv;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TF_CM / 8; ++i) {
      const int cc = sub + 8 * i;
      if (cc < c) {
        float a2 = acc[i];
        for (int j = 0; j < TF_HC; ++j) a2 = fmaf(hs[r][j], wos[cc][j], a2);
        acc[i] = a2;
      }
    }
  }
  if (!live) return;
  const float m = mask ? mask[row] : 1.0f;
#pragma unroll
  for (int i = 0; i < TF_CM / 8; ++i) {
    const int cc = sub + 8 * i;
    if (cc < c) {
      float y = acc[i] * m;
      if (residual) y += x[row * c + cc];
      out[row * c + cc] = y;
    }
  }
}

}  // namespace fpf

extern "C" int fpf_transition_fwd(const FpfTransitionArgs* a, void* stream, char* err, size_t errlen) {
  using namespace fpf;
  FPF_CHECK_VERSION(a);
  if (!a->x || !a->out || !a->w_a || !a->w_b || !a->w_o) return fail(err, errlen, FPF_E_ARGS, "x / out / w_a / w_b / w_o is NULL");
  if (a->rows < 0 || a->c <= 0 || a->hidden <= 0) return fail(err, errlen, FPF_E_SHAPE, "rows=%lld c=%d hidden=%d", (long long)a->rows, a->c, a->hidden);
  if (a->rows == 0) return FPF_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (a->dtype == FPF_DT_BF16) {
    if (a->c != TR_C || a->hidden % TR_HB) return fail(err, errlen, FPF_E_SHAPE, "bf16 transition serves c=128, hidden %% 32 == 0 (got c=%d hidden=%d)", a->c, a->hidden);
    if (!aligned16(a->x) || !aligned16(a->out) || !aligned16(a->w_a) || !aligned16(a->w_b) || !aligned16(a->w_o) ||
        (a->ln_w && !aligned16(a->ln_w)) || (a->ln_b && !aligned16(a->ln_b)))
      return fail(err, errlen, FPF_E_ALIGN, "operands must be 16-byte aligned");
    const int PW = 1;
    const dim3 grid((unsigned)cdiv(a->rows, 32 * TR_WAVES * PW)), block(64 * TR_WAVES);
    hipLaunchKernelGGL((transition_bf16_kernel<PW>), grid, block, 0, st, (const uint16_t*)a->x, (uint16_t*)a->out, a->ln_w, a->ln_b, a->eps,
                       (const uint16_t*)a->w_a, (const uint16_t*)a->w_b, (const uint16_t*)a->w_o, a->row_mask, a->residual, a->rows, a->hidden);
    return launched(err, errlen, "fpf_transition_fwd(bf16)");
  }
  if (a->dtype == FPF_DT_F32) {
    if (a->c > TF_CM) return fail(err, errlen, FPF_E_SHAPE, "fp32 transition serves c <= %d (got %d)", TF_CM, a->c);
    const dim3 grid((unsigned)cdiv(a->rows, TF_R)), block(256);
    hipLaunchKernelGGL(transition_f32_kernel, grid, block, 0, st, (const float*)a->x, (float*)a->out, a->ln_w, a->ln_b, a->eps,
                       (const float*)a->w_a, (const float*)a->w_b, (const float*)a->w_o, a->row_mask, a->residual, a->rows, a->c, a->hidden);
    return launched(err, errlen, "fpf_transition_fwd(f32)");
  }
  return fail(err, errlen, FPF_E_DTYPE, "dtype %d", a->dtype);
}
