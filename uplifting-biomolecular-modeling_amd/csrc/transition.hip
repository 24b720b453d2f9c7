// Fused pair transition: out = [x +] mask * W_o( silu(W_a n) * (W_b n) ), n = LayerNorm(x).
// Replaces common/opt_core/opt_core/kernels/transition/__init__.py:1074 (transition) / attn/pair_fused.py:1519.
//
// bf16 path (c = 128): one wave owns PW x 32 pixel rows.  LN runs in registers and leaves the normalised rows as the
// B operand of v_mfma_f32_32x32x16_bf16 (lane n%32 = pixel, channels 64*(lane/32) + 8t .. +7 for k-step t).  GEMM 1 is
// computed transposed, a^T = W_a n^T, so its D layout (lane = pixel, 16 hidden values) IS the B operand of GEMM 2
// out^T = W_o h^T once the hidden index of each k-step is permuted the same way in W_o: the 4c hidden never leaves the
// registers.  Weights stream through a 3-buffer LDS ring in 32-hidden chunks shared by the 4 waves of a workgroup (the next
// two chunks' transfers are in flight while the current one feeds the MFMAs; one barrier per chunk).  The grid is persistent
// (two workgroups per CU, each walking every grid-th 128-pixel tile) and the ring runs across tiles, so the weight stream
// starts once per workgroup; the kernel holds 241 VGPRs without spills (a workgroup per tile spilled 23 of them, whose
// scratch traffic doubled the kernel's HBM bytes).
// fp32 path (exact tier): c = 128 on the fp32 matrix core (transition_f32_mfma), other widths LDS-tiled scalar FMA.
#include "rowtile.h"

namespace fpf {

constexpr int TR_C = 128;
constexpr int TR_KS = TR_C / 16;      // k-steps of GEMM 1
constexpr int TR_HB = 32;             // hidden rows per chunk
// 32-row tiles per wave and waves per workgroup: 4 waves (one per SIMD) and two workgroups per CU, whose waves share a SIMD
// without sharing a barrier, so one can run its MFMAs while the other evaluates its activation (measured 9-10 % faster than
// 8 waves in one workgroup, and than 2 tiles x 1 wave per SIMD)
constexpr int TR_PW = 1, TR_NW = 4;
constexpr int TR_NBUF = 3;            // weight-chunk ring: 2 chunks in flight (73 KB of LDS per workgroup: two fit a CU)

// The single track's pair bias projected from the written rows (BIAS instances): bias[b, h, i, j] = LN(out row) . w[h, :]
// for out rows of a pair tensor [B, n, n, 128], by the same instructions as the bias output of the tri-att prologue
// (rt_ln on the stored bf16 values, then D = W x^T on the matrix core), so the values equal fpf_apb_bias_fwd's bitwise.
struct TrBias {
  const uint16_t* w;         // [H, 128] bf16
  const float* ln_w;         // [128] or NULL
  const float* ln_b;
  float eps;
  int H;
  int bf16;                  // the bias stored as bf16 (else fp32)
  void* out;                 // [B, H, n, ld]
  int64_t n, ld;
};

// XLN: the GEMM input rows come from xln (the caller's own LayerNorm output of x) as they are; the residual reads x.
template <int PW, int NW, bool XLN, bool BIAS>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2))) transition_bf16_kernel(const uint16_t* x, uint16_t* out, const float* __restrict__ ln_w,
                                                              const float* __restrict__ ln_b, float eps, const uint16_t* __restrict__ wa,
                                                              const uint16_t* __restrict__ wb, const uint16_t* __restrict__ wo,
                                                              const float* __restrict__ mask, int residual, int64_t rows, int hidden,
                                                              const uint16_t* __restrict__ xln, const TrBias zb) {
  // weight chunk hb = W_a / W_b rows hb*32 .. +31 (all 128 inputs) and W_o columns hb*32 .. +31 (all 128 outputs), 24 KB,
  // streamed by DMA (global_load_lds_dwordx4, no VGPR staging) through a ring of TR_NBUF buffers, TR_NBUF - 1 chunks in
  // flight.  W_a / W_b rows are 16 chunks of 16 bytes stored at position c ^ (row & 15) (conflict-free fragment reads of 16
  // consecutive rows); W_o rows are 4 chunks stored at position c ^ ((row >> 2) & 3).
  __shared__ __attribute__((aligned(16))) uint16_t sWa[TR_NBUF][TR_HB * TR_C];
  __shared__ __attribute__((aligned(16))) uint16_t sWb[TR_NBUF][TR_HB * TR_C];
  __shared__ __attribute__((aligned(16))) uint16_t sWo[TR_NBUF][TR_C * TR_HB];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, n = l & 31, g = l >> 5;
  // DMA map: slot sl = tid + 64 NW q of each 512-slot matrix chunk (each wave instruction fills 64 contiguous slots)
  constexpr int NQ = 512 / (64 * NW);
  const int nhb = hidden / TR_HB;
  const int64_t ntiles = cdiv(rows, (int64_t)32 * PW * NW);
  const int nkt = (int)((ntiles - blockIdx.x + gridDim.x - 1) / gridDim.x);   // tiles of this workgroup (the grid is <= ntiles)
  const int U = nkt * nhb;                                                     // weight chunks it streams
  static_assert(TR_NBUF == 3, "the ring indices below step through 3 buffers");
  auto issue = [&](int buf, int hb) {   // chunk hb of the hidden into ring buffer buf
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int sl = tid + 64 * NW * q;
      const int ar = sl >> 4, ac = (sl & 15) ^ (ar & 15);              // W_a / W_b: row, source 16-byte column
      const int orow = sl >> 2, oc = (sl & 3) ^ ((orow >> 2) & 3);     // W_o: row (c_out), source 16-byte column
      const int lslot = (64 * NW * q + 64 * wave) * 8;
      lds_dma16(wa + (int64_t)(hb * TR_HB + ar) * TR_C + ac * 8, lds_addr(&sWa[buf][lslot]));
      lds_dma16(wb + (int64_t)(hb * TR_HB + ar) * TR_C + ac * 8, lds_addr(&sWb[buf][lslot]));
      lds_dma16(wo + (int64_t)orow * hidden + hb * TR_HB + oc * 8, lds_addr(&sWo[buf][lslot]));
    }
  };
  __shared__ __attribute__((aligned(16))) float sLN[2 * RT_C];
  __shared__ __attribute__((aligned(16))) float sLNz[BIAS ? 2 * RT_C : 4];
  rt_stage_affine(sLN, ln_w, ln_b, tid, 64 * NW);
  if constexpr (BIAS) rt_stage_affine(sLNz, zb.ln_w, zb.ln_b, tid, 64 * NW);
  issue(0, 0);
  if (U > 1) issue(1, nhb > 1 ? 1 : 0);
  int buf = 0;                                         // ring buffer of chunk u (u mod 3)
  __syncthreads();                                     // sLN visible
  for (int kt = 0; kt < nkt; ++kt) {
  const int64_t pix0 = ((int64_t)(blockIdx.x + (int64_t)kt * gridDim.x) * NW + wave) * (32 * PW);
  bf16x8 xb[PW][TR_KS];
#pragma unroll
  for (int p = 0; p < PW; ++p) {
    const int64_t pix = pix0 + 32 * p + n;
    u32x4 raw[8];
    rt_load((XLN ? xln : x) + (pix < rows ? pix : 0) * TR_C, pix < rows, g, raw);
    if constexpr (XLN) {
#pragma unroll
      for (int c = 0; c < TR_KS; ++c) xb[p][c] = as_bf8(raw[c]);
    } else {
      rt_ln(raw, g, sLN, eps, xb[p]);
    }
  }
  if (kt == 0) {
    // chunk 0 landed (the row loads above are younger and may still be counted), then published
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
  f32x16 acc[PW][4];
#pragma unroll
  for (int p = 0; p < PW; ++p)
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) acc[p][cb] = f32x16{};
  for (int hb = 0; hb < nhb; ++hb) {
    const int u = kt * nhb + hb;
    if (u + 2 < U) {                                   // chunk u + 2: its buffer held chunk u - 1, finished before the last barrier
      const int h2 = hb + 2;
      issue(buf == 0 ? 2 : buf - 1, h2 < nhb ? h2 : (h2 - nhb < nhb ? h2 - nhb : 0));
    }
    f32x16 a[PW], b[PW];
#pragma unroll
    for (int p = 0; p < PW; ++p) {
      a[p] = f32x16{};
      b[p] = f32x16{};
    }
    const uint16_t* ra = &sWa[buf][n * TR_C];
    const uint16_t* rb = &sWb[buf][n * TR_C];
    auto wfrag = [&](const uint16_t* r, int t) { return as_bf8(*reinterpret_cast<const u32x4*>(r + 8 * (rt_chunk(t, g) ^ (n & 15)))); };
    bf16x8 fa = wfrag(ra, 0), fb = wfrag(rb, 0);
#pragma unroll
    for (int t = 0; t < TR_KS; ++t) {
      const bf16x8 ca = fa, cbf = fb;
      if (t + 1 < TR_KS) {                      // one k-step of fragment lookahead
        fa = wfrag(ra, t + 1);
        fb = wfrag(rb, t + 1);
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
      const int orr = cb * 32 + n, sw = (orr >> 2) & 3;
      const uint16_t* wrow = &sWo[buf][orr * TR_HB];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        // hidden 16s + 4g + 0..3 (chunk 2s, bytes 8g) and 16s + 8 + 4g + 0..3 (chunk 2s + 1)
        const u32x2 lo = *reinterpret_cast<const u32x2*>(wrow + 8 * ((2 * s) ^ sw) + 4 * g);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(wrow + 8 * ((2 * s + 1) ^ sw) + 4 * g);
        const bf16x8 fo = as_bf8(u32x4{lo[0], lo[1], hi[0], hi[1]});
#pragma unroll
        for (int p = 0; p < PW; ++p) acc[p][cb] = mfma32(fo, hf[p][s], acc[p][cb]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (u + 1 < U) {                             // chunk u + 1 landed: only chunk u + 2's transfers (3 NQ) may be outstanding
      static_assert(TR_NBUF == 3, "the waits below count one chunk in flight behind the awaited one");
      if constexpr (NQ == 1) {
        if (u + 2 < U) asm volatile("s_waitcnt vmcnt(3)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      } else {
        static_assert(NQ == 2, "4 or 8 waves");
        if (u + 2 < U) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      __builtin_amdgcn_s_barrier();
    }
    buf = buf == 2 ? 0 : buf + 1;
  }
  // epilogue: lane (pixel n, half g) holds c_out = 32 cb + c_row(v, g); after the lane exchange it holds channels
  // 32 cb + 8g .. +7 and 32 cb + 16 + 8g .. +7, stored (with mask and residual) in 16-byte pieces
#pragma unroll
  for (int p = 0; p < PW; ++p) {
    const int64_t pix = pix0 + 32 * p + n;
    const bool live = pix < rows;
    const float m = (mask && live) ? mask[pix] : 1.0f;
    u32x4 zo[8];                                       // the written row, chunk 2 cb + h2 = channels 32 cb + 16 h2 + 8 g .. +7
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      float y[16];
      rt_regroup_f32(acc[p][cb], y);
      if (!live) {
        zo[2 * cb] = zo[2 * cb + 1] = u32x4{0, 0, 0, 0};
        continue;
      }
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
        const u32x4 w = u32x4{pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7])};
        *reinterpret_cast<u32x4*>(out + c0) = w;
        zo[2 * cb + h2] = w;
      }
    }
    if constexpr (BIAS) {
      // chunk 2 cb + h2 of the lane is rt_chunk(2 cb + h2, g): zo is the row in the order rt_load gives the prologue.  The
      // lane index is re-read here (opaque_lane): weight addresses derived from it and hoisted out of the tile loop would
      // hold registers the chunk loop needs
      __builtin_amdgcn_sched_barrier(0);               // the output stores above are issued; nothing of this moves above them
      const int ol = opaque_lane(), on = ol & 31;
      bf16x8 xn[8];
      rt_ln(zo, g, sLNz, zb.eps, xn);
      f32x16 bacc = {};
      const uint16_t* wrow = zb.w + on * TR_C + 8 * g;
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const u32x4 wv = on < zb.H ? *reinterpret_cast<const u32x4*>(wrow + 16 * t) : u32x4{0, 0, 0, 0};
        bacc = mfma32(as_bf8(wv), xn[t], bacc);
      }
      if (live) {
        // head c_row(v, g) of pixel (b, i, j): offset base + head * (n ld); the head rows come from the re-read lane index
        const int64_t nn = zb.n * zb.n, b = pix / nn, rem = pix - b * nn, i = rem / zb.n, j = rem - i * zb.n;
        const int64_t hs = zb.n * zb.ld, base = (b * zb.H * zb.n + i) * zb.ld + j;
        const int og = ol >> 5;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int hh = c_row(v, og);
          if (hh >= zb.H) continue;
          const int64_t o = base + hh * hs;
          if (zb.bf16) reinterpret_cast<uint16_t*>(zb.out)[o] = f2bf(bacc[v] * 1.0f);
          else reinterpret_cast<float*>(zb.out)[o] = bacc[v] * 1.0f;
        }
      }
    }
  }
  }
}

// ---------------------------------------------------------------------------------------------------------------- fp32 (exact tier)
constexpr int TF_R = 32;    // rows per workgroup
constexpr int TF_HC = 16;   // hidden per chunk
constexpr int TF_CM = 384;  // max c (the single track's c_s; the pair track's 128 takes the narrow instance)

// CM: the widest c an instance serves (LDS tiles [TF_R][CM + 1] of x and [TF_HC][CM + 1] of W_a, W_b)
template <int CM>
__global__ void __launch_bounds__(256) transition_f32_kernel(const float* x, float* out, const float* __restrict__ ln_w,
                                                             const float* __restrict__ ln_b, float eps, const float* __restrict__ wa,
                                                             const float* __restrict__ wb, const float* __restrict__ wo,
                                                             const float* __restrict__ mask, int residual, int64_t rows, int c, int hidden) {
  __shared__ float xs[TF_R][CM + 1];
  __shared__ float was[TF_HC][CM + 1];
  __shared__ float wbs[TF_HC][CM + 1];
  __shared__ float wos[CM][TF_HC + 1];
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
  float acc[CM / 8];
#pragma unroll
  for (int i = 0; i < CM / 8; ++i) acc[i] = 0.f;
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
    for (int i = 0; i < CM / 8; ++i) {
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
  for (int i = 0; i < CM / 8; ++i) {
    const int cc = sub + 8 * i;
    if (cc < c) {
      float y = acc[i] * m;
      if (residual) y += x[row * c + cc];
      out[row * c + cc] = y;
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------- fp32, c = 128 (exact tier)
// The bf16 kernel's structure on the fp32 matrix core (v_mfma_f32_32x32x2_f32: fp32 operands, fp32 products and sums).  One
// wave owns 32 pixel rows; lane (n, g) holds pixel n's LayerNorm'd channels 64 g .. 64 g + 63, so k-step s of GEMM 1 pairs
// channels s (g = 0) and 64 + s (g = 1) -- each lane's weight fragment is then 4 consecutive k-steps in one 16-byte LDS
// read.  GEMM 1 is computed transposed (a^T = W_a n^T: lane = pixel, 16 hidden rows per lane), and k-step t of GEMM 2
// pairs the hidden rows register t holds in the two lane halves, so h = silu(a) * b feeds GEMM 2 from the registers it was
// computed in.  Weights stream through two LDS buffers in 32-hidden chunks shared by the 8 waves (the next chunk's global
// loads are issued before the current chunk's MFMAs and stored after them; one barrier per chunk).
constexpr int TX_HB = 32;             // hidden rows per chunk
constexpr int TX_NW = 8;              // waves per workgroup
constexpr int TX_WP = RTF_WP;         // LDS pitch (floats) of a W_a / W_b chunk row: 16 consecutive rows on distinct banks
constexpr int TX_OP = TX_HB + 4;      // LDS pitch of a W_o chunk row (one output channel)

__global__ void __launch_bounds__(64 * TX_NW) transition_f32_mfma(const float* x, float* out, const float* __restrict__ ln_w,
                                                                  const float* __restrict__ ln_b, float eps, const float* __restrict__ wa,
                                                                  const float* __restrict__ wb, const float* __restrict__ wo,
                                                                  const float* __restrict__ mask, int residual, int64_t rows, int hidden) {
  __shared__ __attribute__((aligned(16))) float sWa[2][TX_HB * TX_WP];
  __shared__ __attribute__((aligned(16))) float sWb[2][TX_HB * TX_WP];
  __shared__ __attribute__((aligned(16))) float sWo[2][TR_C * TX_OP];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, n = l & 31, g = l >> 5;
  const int64_t pix = ((int64_t)blockIdx.x * TX_NW + wave) * 32 + n;
  const bool live = pix < rows;
  // chunk hb: W_a / W_b rows hb 32 .. + 31 (1024 float4 each) and W_o columns hb 32 .. + 31 of all 128 rows (1024 float4);
  // thread tid moves float4 tid and tid + 512 of each
  f32x4 stage[6];
  auto gload = [&](int hb) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int i = tid + 64 * TX_NW * q;
      const int64_t wrow = (int64_t)(hb * TX_HB + (i >> 5)) * TR_C + (i & 31) * 4;
      stage[q] = *reinterpret_cast<const f32x4*>(wa + wrow);
      stage[2 + q] = *reinterpret_cast<const f32x4*>(wb + wrow);
      stage[4 + q] = *reinterpret_cast<const f32x4*>(wo + (int64_t)(i >> 3) * hidden + hb * TX_HB + (i & 7) * 4);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int i = tid + 64 * TX_NW * q;
      *reinterpret_cast<f32x4*>(&sWa[buf][(i >> 5) * TX_WP + (i & 31) * 4]) = stage[q];
      *reinterpret_cast<f32x4*>(&sWb[buf][(i >> 5) * TX_WP + (i & 31) * 4]) = stage[2 + q];
      *reinterpret_cast<f32x4*>(&sWo[buf][(i >> 3) * TX_OP + (i & 7) * 4]) = stage[4 + q];
    }
  };
  const int nhb = hidden / TX_HB;
  gload(0);
  float xn[64];                                  // the lane's LayerNorm'd half of its pixel row
  rtf_ln(x + (live ? pix : 0) * TR_C, live, g, ln_w, ln_b, eps, xn);
  lstore(0);
  __syncthreads();
  f32x16 acc[4];
#pragma unroll
  for (int cb = 0; cb < 4; ++cb) acc[cb] = f32x16{};
  for (int hb = 0; hb < nhb; ++hb) {
    const int buf = hb & 1;
    if (hb + 1 < nhb) gload(hb + 1);
    f32x16 ab[2] = {f32x16{}, f32x16{}};
    const float* const wab[2] = {&sWa[buf][n * TX_WP + 64 * g], &sWb[buf][n * TX_WP + 64 * g]};
    rtf_gemm<2>(wab, xn, ab);
    f32x16& a = ab[0];
    const f32x16& b = ab[1];
    // h = silu(a) * b in place of a; register t holds hidden row 8 (t / 4) + 4 g + t % 4 of the chunk
#pragma unroll
    for (int v = 0; v < 16; ++v) a[v] = a[v] / (1.0f + expf(-a[v])) * b[v];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f32x4 fo[4];
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) fo[cb] = *reinterpret_cast<const f32x4*>(&sWo[buf][(32 * cb + n) * TX_OP + 4 * g + 8 * q]);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) acc[cb] = mfma32f(fo[cb][e], a[4 * q + e], acc[cb]);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (hb + 1 < nhb) {
      lstore(buf ^ 1);                           // its previous chunk (hb - 1) was read by every wave before the last barrier
      __syncthreads();
    }
  }
  if (!live) return;
  const float m = mask ? mask[pix] : 1.0f;
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t o = pix * TR_C + 32 * cb + 8 * q + 4 * g;      // channels of registers 4 q .. 4 q + 3
      f32x4 y;
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = acc[cb][4 * q + e] * m;
      if (residual) {
        const f32x4 r = *reinterpret_cast<const f32x4*>(x + o);
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] += r[e];
      }
      *reinterpret_cast<f32x4*>(out + o) = y;
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
    if (a->x_ln && !aligned16(a->x_ln)) return fail(err, errlen, FPF_E_ALIGN, "x_ln must be 16-byte aligned");
    TrBias zb = {};
    if (a->w_z) {
      if (!a->z_bias) return fail(err, errlen, FPF_E_ARGS, "w_z given without z_bias");
      if (a->z_heads < 1 || a->z_heads > 32) return fail(err, errlen, FPF_E_SHAPE, "z_heads %d outside 1 .. 32", a->z_heads);
      if (a->pair_n <= 0 || a->rows % (a->pair_n * a->pair_n) != 0)
        return fail(err, errlen, FPF_E_SHAPE, "the pair bias needs rows = B N N (rows %lld, pair_n %lld)", (long long)a->rows, (long long)a->pair_n);
      if (!(a->z_bias_dtype == FPF_DT_F32 || a->z_bias_dtype == FPF_DT_BF16)) return fail(err, errlen, FPF_E_DTYPE, "z_bias_dtype %d", a->z_bias_dtype);
      const int64_t ld = a->z_bias_ld > 0 ? a->z_bias_ld : a->pair_n;
      if (ld < a->pair_n) return fail(err, errlen, FPF_E_SHAPE, "z_bias_ld %lld < N %lld", (long long)ld, (long long)a->pair_n);
      if (!aligned16(a->w_z) || (a->z_ln_w && !aligned16(a->z_ln_w)) || (a->z_ln_b && !aligned16(a->z_ln_b)))
        return fail(err, errlen, FPF_E_ALIGN, "w_z / z_ln_w / z_ln_b must be 16-byte aligned");
      zb = TrBias{(const uint16_t*)a->w_z, a->z_ln_w, a->z_ln_b, a->z_eps, a->z_heads, a->z_bias_dtype == FPF_DT_BF16, a->z_bias, a->pair_n, ld};
    } else if (a->z_bias) {
      return fail(err, errlen, FPF_E_ARGS, "z_bias given without w_z");
    }
    constexpr int PW = TR_PW, NW = TR_NW;
    const dim3 grid((unsigned)std::min<int64_t>(cdiv(a->rows, 32 * NW * PW), 2 * (int64_t)num_cus())), block(64 * NW);
    const bool xl = a->x_ln != nullptr, bz = a->w_z != nullptr;
    auto k = xl ? (bz ? transition_bf16_kernel<PW, NW, true, true> : transition_bf16_kernel<PW, NW, true, false>)
                : (bz ? transition_bf16_kernel<PW, NW, false, true> : transition_bf16_kernel<PW, NW, false, false>);
    hipLaunchKernelGGL(k, grid, block, 0, st, (const uint16_t*)a->x, (uint16_t*)a->out, a->ln_w, a->ln_b, a->eps, (const uint16_t*)a->w_a,
                       (const uint16_t*)a->w_b, (const uint16_t*)a->w_o, a->row_mask, a->residual, a->rows, a->hidden, (const uint16_t*)a->x_ln, zb);
    return launched(err, errlen, "fpf_transition_fwd(bf16)");
  }
  if (a->dtype == FPF_DT_F32) {
    if (a->x_ln) return fail(err, errlen, FPF_E_DTYPE, "x_ln serves the bf16 transition");
    if (a->w_z || a->z_bias) return fail(err, errlen, FPF_E_DTYPE, "the pair bias serves the bf16 transition");
    if (a->c > TF_CM) return fail(err, errlen, FPF_E_SHAPE, "fp32 transition serves c <= %d (got %d)", TF_CM, a->c);
    if (a->c == TR_C && a->hidden % TX_HB == 0 && aligned16(a->x) && aligned16(a->out) && aligned16(a->w_a) && aligned16(a->w_b) &&
        aligned16(a->w_o) && (!a->ln_w || aligned16(a->ln_w)) && (!a->ln_b || aligned16(a->ln_b))) {   // the matrix-core kernel
      const dim3 grid((unsigned)cdiv(a->rows, 32 * TX_NW)), block(64 * TX_NW);
      hipLaunchKernelGGL(transition_f32_mfma, grid, block, 0, st, (const float*)a->x, (float*)a->out, a->ln_w, a->ln_b, a->eps,
                         (const float*)a->w_a, (const float*)a->w_b, (const float*)a->w_o, a->row_mask, a->residual, a->rows, a->hidden);
      return launched(err, errlen, "fpf_transition_fwd(f32 mfma)");
    }
    const dim3 grid((unsigned)cdiv(a->rows, TF_R)), block(256);
    if (a->c <= 128)
      hipLaunchKernelGGL(transition_f32_kernel<128>, grid, block, 0, st, (const float*)a->x, (float*)a->out, a->ln_w, a->ln_b, a->eps,
                         (const float*)a->w_a, (const float*)a->w_b, (const float*)a->w_o, a->row_mask, a->residual, a->rows, a->c, a->hidden);
    else
      hipLaunchKernelGGL(transition_f32_kernel<TF_CM>, grid, block, 0, st, (const float*)a->x, (float*)a->out, a->ln_w, a->ln_b, a->eps,
                         (const float*)a->w_a, (const float*)a->w_b, (const float*)a->w_o, a->row_mask, a->residual, a->rows, a->c, a->hidden);
    return launched(err, errlen, "fpf_transition_fwd(f32)");
  }
  return fail(err, errlen, FPF_E_DTYPE, "dtype %d", a->dtype);
}
