// Fused pair transition: out = [x +] mask * W_o( silu(W_a n) * (W_b n) ), n = LayerNorm(x).
// Replaces common/opt_core/opt_core/kernels/transition/__init__.py:1074 (transition) / attn/pair_fused.py:1519.
//
// bf16 path (c = 128): one wave owns PW x 32 pixel rows.  LN runs in registers and leaves the normalised rows as the
// B operand of v_mfma_f32_32x32x16_bf16 (lane n%32 = pixel, channels 64*(lane/32) + 8t .. +7 for k-step t).  GEMM 1 is
// computed transposed, a^T = W_a n^T, so its D layout (lane = pixel, 16 hidden values) IS the B operand of GEMM 2
// out^T = W_o h^T once the hidden index of each k-step is permuted the same way in W_o: the 4c hidden never leaves the
// registers.  Weights stream through LDS in 32-hidden chunks shared by the 4 waves of a workgroup.
// fp32 path (exact tier): LDS-tiled scalar FMA, fp32 throughout.
#include "fpf_common.h"

namespace fpf {

constexpr int TR_C = 128;
constexpr int TR_KS = TR_C / 16;      // k-steps of GEMM 1
constexpr int TR_HB = 32;             // hidden rows per chunk
constexpr int TR_WLD = TR_C + 8;      // LDS pitch of a W_a / W_b chunk row (bf16): 272 B, conflict-free 16-byte reads
constexpr int TR_OLD = TR_HB + 4;     // LDS pitch of a W_o chunk row (bf16): 72 B, conflict-free 8-byte reads

// Loads 32 pixel rows of 128 bf16 (lane: pixel n, channel half g) and returns LN(x) as 8 B-operand fragments.
__device__ __forceinline__ void ln128_fragments(const uint16_t* __restrict__ xrow, bool live, int g, const float* __restrict__ ln_w,
                                                const float* __restrict__ ln_b, float eps, bf16x8 (&xb)[TR_KS]) {
  float xv[64];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    u32x4 r = live ? *reinterpret_cast<const u32x4*>(xrow + 64 * g + 8 * t) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xv[8 * t + 2 * e] = lo_bf(r[e]);
      xv[8 * t + 2 * e + 1] = hi_bf(r[e]);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 64; ++i) s += xv[i];
  s = half_sum(s);
  const float mean = s * (1.0f / 128.0f);
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    const float d = xv[i] - mean;
    q += d * d;
  }
  q = half_sum(q);
  const float rstd = 1.0f / sqrtf(q * (1.0f / 128.0f) + eps);
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int c0 = 64 * g + 8 * t;
    f32x4 w0 = ln_w ? *reinterpret_cast<const f32x4*>(ln_w + c0) : f32x4{1, 1, 1, 1};
    f32x4 w1 = ln_w ? *reinterpret_cast<const f32x4*>(ln_w + c0 + 4) : f32x4{1, 1, 1, 1};
    f32x4 b0 = ln_b ? *reinterpret_cast<const f32x4*>(ln_b + c0) : f32x4{0, 0, 0, 0};
    f32x4 b1 = ln_b ? *reinterpret_cast<const f32x4*>(ln_b + c0 + 4) : f32x4{0, 0, 0, 0};
    float y[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      y[e] = (xv[8 * t + e] - mean) * rstd * w0[e] + b0[e];
      y[4 + e] = (xv[8 * t + 4 + e] - mean) * rstd * w1[e] + b1[e];
    }
    xb[t] = as_bf8(u32x4{pack2(y[0], y[1]), pack2(y[2], y[3]), pack2(y[4], y[5]), pack2(y[6], y[7])});
  }
}

template <int PW>
__global__ void __launch_bounds__(256) transition_bf16_kernel(const uint16_t* x, uint16_t* out, const float* __restrict__ ln_w,
                                                              const float* __restrict__ ln_b, float eps, const uint16_t* __restrict__ wa,
                                                              const uint16_t* __restrict__ wb, const uint16_t* __restrict__ wo,
                                                              const float* __restrict__ mask, int residual, int64_t rows, int hidden) {
  __shared__ __attribute__((aligned(16))) uint16_t sWa[TR_HB * TR_WLD];
  __shared__ __attribute__((aligned(16))) uint16_t sWb[TR_HB * TR_WLD];
  __shared__ __attribute__((aligned(16))) uint16_t sWo[TR_C * TR_OLD];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, n = l & 31, g = l >> 5;
  const int64_t pix0 = ((int64_t)blockIdx.x * 4 + wave) * (32 * PW);

  bf16x8 xb[PW][TR_KS];
#pragma unroll
  for (int p = 0; p < PW; ++p) {
    const int64_t pix = pix0 + 32 * p + n;
    ln128_fragments(x + pix * TR_C, pix < rows, g, ln_w, ln_b, eps, xb[p]);
  }
  f32x16 acc[PW][4];
#pragma unroll
  for (int p = 0; p < PW; ++p)
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) acc[p][cb] = f32x16{};

  const int nhb = hidden / TR_HB;
  for (int hb = 0; hb < nhb; ++hb) {
    __syncthreads();
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int i = tid + 256 * it;
      const int r = i >> 4, ch = i & 15;
      const int64_t src = (int64_t)(hb * TR_HB + r) * TR_C + ch * 8;
      *reinterpret_cast<u32x4*>(&sWa[r * TR_WLD + ch * 8]) = *reinterpret_cast<const u32x4*>(wa + src);
      *reinterpret_cast<u32x4*>(&sWb[r * TR_WLD + ch * 8]) = *reinterpret_cast<const u32x4*>(wb + src);
      const int ro = i >> 2, co = i & 3;
      const u32x4 w = *reinterpret_cast<const u32x4*>(wo + (int64_t)ro * hidden + hb * TR_HB + co * 8);
      *reinterpret_cast<u32x2*>(&sWo[ro * TR_OLD + co * 8]) = u32x2{w[0], w[1]};
      *reinterpret_cast<u32x2*>(&sWo[ro * TR_OLD + co * 8 + 4]) = u32x2{w[2], w[3]};
    }
    __syncthreads();
    f32x16 a[PW], b[PW];
#pragma unroll
    for (int p = 0; p < PW; ++p) {
      a[p] = f32x16{};
      b[p] = f32x16{};
    }
#pragma unroll
    for (int t = 0; t < TR_KS; ++t) {
      const bf16x8 fa = as_bf8(*reinterpret_cast<const u32x4*>(&sWa[n * TR_WLD + 64 * g + 8 * t]));
      const bf16x8 fb = as_bf8(*reinterpret_cast<const u32x4*>(&sWb[n * TR_WLD + 64 * g + 8 * t]));
#pragma unroll
      for (int p = 0; p < PW; ++p) {
        a[p] = mfma32(fa, xb[p][t], a[p]);
        b[p] = mfma32(fb, xb[p][t], b[p]);
      }
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
          const float h0 = a0 / (1.0f + __expf(-a0)) * b[p][v0];
          const float h1 = a1 / (1.0f + __expf(-a1)) * b[p][v0 + 1];
          w[e] = pack2(h0, h1);
        }
        hf[p][s] = as_bf8(u32x4{w[0], w[1], w[2], w[3]});
      }
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const uint16_t* wrow = &sWo[(cb * 32 + n) * TR_OLD + 16 * s + 4 * g];
        const u32x2 lo = *reinterpret_cast<const u32x2*>(wrow);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(wrow + 8);
        const bf16x8 fo = as_bf8(u32x4{lo[0], lo[1], hi[0], hi[1]});
#pragma unroll
        for (int p = 0; p < PW; ++p) acc[p][cb] = mfma32(fo, hf[p][s], acc[p][cb]);
      }
  }
  // epilogue: lane (pixel n, half g) holds c_out = 32 cb + 8 q + 4 g + 0..3 in registers 4q .. 4q+3
#pragma unroll
  for (int p = 0; p < PW; ++p) {
    const int64_t pix = pix0 + 32 * p + n;
    if (pix >= rows) continue;
    const float m = mask ? mask[pix] : 1.0f;
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c0 = 32 * cb + 8 * q + 4 * g;
        float y0 = acc[p][cb][4 * q] * m, y1 = acc[p][cb][4 * q + 1] * m, y2 = acc[p][cb][4 * q + 2] * m, y3 = acc[p][cb][4 * q + 3] * m;
        if (residual) {
          const u32x2 r = *reinterpret_cast<const u32x2*>(x + pix * TR_C + c0);
          y0 += lo_bf(r[0]);
          y1 += hi_bf(r[0]);
          y2 += lo_bf(r[1]);
          y3 += hi_bf(r[1]);
        }
        *reinterpret_cast<u32x2*>(out + pix * TR_C + c0) = u32x2{pack2(y0, y1), pack2(y2, y3)};
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
    const dim3 grid((unsigned)cdiv(a->rows, 128 * PW)), block(256);
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
