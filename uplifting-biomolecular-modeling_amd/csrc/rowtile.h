// Device building blocks of the persistent "32 pixel rows x 128 channels -> LayerNorm -> MFMA against LDS-resident weights"
// kernels (trimul K1 / K3, tri-att prologue / epilogue).  One wave owns a tile of 32 pixel rows at a time and walks the
// tile list on its own: weights are staged in LDS once per workgroup, so the tile loop has no workgroup barrier and the
// 8 waves of a workgroup (2 per SIMD) overlap each other's loads, LayerNorm and MFMA.
//
// Operand layout (v_mfma_f32_32x32x16_bf16, lane = 32 * g + n): the normalised rows are the B operand -- lane (n, g) holds
// pixel n's channels 16t + 8g .. +7 for k-step t -- and the weight rows (W[out][in], LDS pitch RT_LD) are the A operand
// read at the same channel offsets, so D = W x^T comes out with lane (n, g) holding pixel n and the 16 output channels
// c_row(v, g) of a 32-channel block.
#pragma once
#include "fpf_common.h"

namespace fpf {

constexpr int RT_C = 128;            // channels per pixel row
constexpr int RT_LD = RT_C + 8;      // LDS pitch (bf16) of a 128-wide weight row: 272 B, conflict-free 16-byte reads
constexpr int RT_WAVES = 8;          // waves per workgroup

// Tile t of a persistent loop's [B][rows][tpr] list of 32-pixel tiles: image b, row r, column tile c.  32-bit division (the
// launchers refuse lists of 2^31 tiles or more: rt_tiles_ok); t, per_b and tpr are wave-uniform, so this is scalar code.
struct RtTile {
  int64_t b, r, c;
};
__device__ __forceinline__ RtTile rt_tile(uint32_t t, uint32_t per_b, uint32_t tpr) {
  const uint32_t b = t / per_b, rem = t - b * per_b, r = rem / tpr;
  return {(int64_t)b, (int64_t)r, (int64_t)(rem - r * tpr)};
}
inline bool rt_tiles_ok(int64_t tiles) { return tiles >= 0 && tiles < (int64_t(1) << 31); }

// K-step t of a 128-channel reduction takes channels 16 t .. 16 t + 15: lane (n, g) holds the 8-channel chunk 2 t + g.  The two
// lanes of a pixel read adjacent chunks, so each 16-byte load instruction touches one 32-byte piece of 32 pixel rows.
__device__ __forceinline__ constexpr int rt_chunk(int t, int g) { return 2 * t + g; }

// Raw 16-byte loads of one lane's half of a 128-channel bf16 pixel row (zeros when !live).
__device__ __forceinline__ void rt_load(const uint16_t* __restrict__ row, bool live, int g, u32x4 (&raw)[8]) {
#pragma unroll
  for (int t = 0; t < 8; ++t) raw[t] = live ? *reinterpret_cast<const u32x4*>(row + 8 * rt_chunk(t, g)) : u32x4{0, 0, 0, 0};
}

// The same half row read from fp32 storage and rounded to bf16 (round to nearest even), the compute input of the
// fp32-resident form: a kernel reading it sees exactly the bf16 copy of the row.
__device__ __forceinline__ void rt_load_f32(const float* __restrict__ row, bool live, int g, u32x4 (&raw)[8]) {
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const f32x4 a = live ? *reinterpret_cast<const f32x4*>(row + 8 * rt_chunk(t, g)) : f32x4{0.f, 0.f, 0.f, 0.f};
    const f32x4 b = live ? *reinterpret_cast<const f32x4*>(row + 8 * rt_chunk(t, g) + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
    raw[t] = u32x4{pack2(a[0], a[1]), pack2(a[2], a[3]), pack2(b[0], b[1]), pack2(b[2], b[3])};
  }
}

// LayerNorm over the 128 channels split across lanes n and n + 32 (fp32 statistics, two-pass variance), packed to bf16
// B-operand fragments.  gb = the affine parameters staged in LDS as fp32 [gamma 128 | beta 128] (rt_stage_affine).
__device__ __forceinline__ void rt_ln(const u32x4 (&raw)[8], int g, const float* __restrict__ gb, float eps, bf16x8 (&xb)[8]) {
  float s = 0.f;
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) s += lo_bf(raw[t][e]) + hi_bf(raw[t][e]);
  const float mean = half_sum(s) * (1.0f / 128.0f);
  float q = 0.f;
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float d0 = lo_bf(raw[t][e]) - mean, d1 = hi_bf(raw[t][e]) - mean;
      q += d0 * d0 + d1 * d1;
    }
  const float rstd = 1.0f / sqrtf(half_sum(q) * (1.0f / 128.0f) + eps);
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int c0 = 8 * rt_chunk(t, g);
    const f32x4 w0 = *reinterpret_cast<const f32x4*>(gb + c0), w1 = *reinterpret_cast<const f32x4*>(gb + c0 + 4);
    const f32x4 b0 = *reinterpret_cast<const f32x4*>(gb + RT_C + c0), b1 = *reinterpret_cast<const f32x4*>(gb + RT_C + c0 + 4);
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      o[e] = pack2((lo_bf(raw[t][e]) - mean) * rstd * w0[2 * e] + b0[2 * e], (hi_bf(raw[t][e]) - mean) * rstd * w0[2 * e + 1] + b0[2 * e + 1]);
      o[2 + e] = pack2((lo_bf(raw[t][2 + e]) - mean) * rstd * w1[2 * e] + b1[2 * e],
                       (hi_bf(raw[t][2 + e]) - mean) * rstd * w1[2 * e + 1] + b1[2 * e + 1]);
    }
    xb[t] = as_bf8(u32x4{o[0], o[1], o[2], o[3]});
  }
}

// Stages LayerNorm gamma / beta (NULL = 1 / 0) as fp32 [gamma 128 | beta 128] in LDS.
__device__ __forceinline__ void rt_stage_affine(float* __restrict__ s, const float* __restrict__ w, const float* __restrict__ b, int tid, int nthr) {
  for (int i = tid; i < 2 * RT_C; i += nthr) s[i] = i < RT_C ? (w ? w[i] : 1.0f) : (b ? b[i - RT_C] : 0.0f);
}

// Cooperative copy of `rows` rows of a [rows x 128] bf16 weight matrix into LDS (pitch RT_LD); rows >= valid are zero.
__device__ __forceinline__ void rt_stage_weights(uint16_t* __restrict__ s, const uint16_t* __restrict__ w, int rows, int valid, int tid, int nthr) {
  for (int i = tid; i < rows * 16; i += nthr) {
    const int r = i >> 4, ch = i & 15;
    *reinterpret_cast<u32x4*>(&s[r * RT_LD + ch * 8]) = r < valid ? *reinterpret_cast<const u32x4*>(w + (int64_t)r * RT_C + ch * 8) : u32x4{0, 0, 0, 0};
  }
}

// D = W[row0 .. row0 + 31] x^T over the 128 channels (8 k-steps), weights from LDS.  The weight fragments run LA k-steps
// ahead of the MFMAs (a single MFMA covers ~32 cycles, an LDS read under load ~100), so the matrix core does not wait on
// the reads; LA + 1 fragments are live at a time.
template <int LA = 3, bool XW = false>
__device__ __forceinline__ f32x16 rt_gemm32_la(const uint16_t* __restrict__ s, int row0, int n, int g, const bf16x8 (&xb)[8]) {
  const uint16_t* r = s + (row0 + n) * RT_LD + 8 * g;
  f32x16 acc = {};
  bf16x8 w[8];
#pragma unroll
  for (int t = 0; t < LA; ++t) w[t] = as_bf8(*reinterpret_cast<const u32x4*>(r + 16 * t));
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    if (t + LA < 8) w[t + LA] = as_bf8(*reinterpret_cast<const u32x4*>(r + 16 * (t + LA)));
    acc = XW ? mfma32(xb[t], w[t], acc) : mfma32(w[t], xb[t], acc);
    __builtin_amdgcn_sched_barrier(0);   // keep the read ring as written: bounded register pressure
  }
  return acc;
}
__device__ __forceinline__ f32x16 rt_gemm32(const uint16_t* __restrict__ s, int row0, int n, int g, const bf16x8 (&xb)[8]) {
  return rt_gemm32_la<3, false>(s, row0, n, g, xb);
}

// The swapped product D = x W[row0 .. row0 + 31]^T (same fragments, operands exchanged): lane (n, g) then holds output
// channel row0 + n for the 16 pixels c_row(v, g) of the tile.
__device__ __forceinline__ f32x16 rt_gemm32_xw(const uint16_t* __restrict__ s, int row0, int n, int g, const bf16x8 (&xb)[8]) {
  return rt_gemm32_la<3, true>(s, row0, n, g, xb);
}

// K GEMMs over the same B operand, k-step-major (the K weight fragments of k-step t + 1 are read while the K MFMAs of
// k-step t issue).
template <int K>
__device__ __forceinline__ void rt_gemm32_multi(const uint16_t* const (&s)[K], int row0, int n, int g, const bf16x8 (&xb)[8], f32x16 (&acc)[K]) {
  bf16x8 a[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    acc[k] = f32x16{};
    a[k] = as_bf8(*reinterpret_cast<const u32x4*>(s[k] + (row0 + n) * RT_LD + 8 * g));
  }
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    bf16x8 an[K];
#pragma unroll
    for (int k = 0; k < K; ++k) an[k] = t < 7 ? as_bf8(*reinterpret_cast<const u32x4*>(s[k] + (row0 + n) * RT_LD + 8 * rt_chunk(t + 1, g))) : a[k];
#pragma unroll
    for (int k = 0; k < K; ++k) acc[k] = mfma32(a[k], xb[t], acc[k]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < K; ++k) a[k] = an[k];
  }
}

// The swapped form of rt_gemm32_multi: D_k = x W_k[row0 .. row0 + 31]^T, lane (n, g) holding output channel row0 + n for the
// 16 pixels c_row(v, g).
template <int K>
__device__ __forceinline__ void rt_gemm32_multi_xw(const uint16_t* const (&s)[K], int row0, int n, int g, const bf16x8 (&xb)[8], f32x16 (&acc)[K]) {
  bf16x8 a[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    acc[k] = f32x16{};
    a[k] = as_bf8(*reinterpret_cast<const u32x4*>(s[k] + (row0 + n) * RT_LD + 8 * g));
  }
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    bf16x8 an[K];
#pragma unroll
    for (int k = 0; k < K; ++k) an[k] = t < 7 ? as_bf8(*reinterpret_cast<const u32x4*>(s[k] + (row0 + n) * RT_LD + 8 * rt_chunk(t + 1, g))) : a[k];
#pragma unroll
    for (int k = 0; k < K; ++k) acc[k] = mfma32(xb[t], a[k], acc[k]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < K; ++k) a[k] = an[k];
  }
}

// Repacks a 32 x 32 D fragment (lane (n, g) holds rows c_row(v, g) of column n) into bf16 16-byte chunks: afterwards lane
// (n, g) holds rows 8g .. 8g + 7 (lo) and 16 + 8g .. 16 + 8g + 7 (hi) of column n.  Lanes n and n + 32 trade the four-row
// groups the other one needs with v_permlane32_swap (swap(A, B) exchanges A's upper half-wave with B's lower half-wave),
// so a pixel's 32 consecutive channels leave in two 16-byte stores instead of four 8-byte ones.
__device__ __forceinline__ void rt_pack16(const f32x16& acc, u32x4& lo, u32x4& hi) {
  uint32_t p[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) p[e] = pack2(acc[2 * e], acc[2 * e + 1]);
  // p[0], p[1]: rows 4g + 0..3;  p[2], p[3]: rows 8 + 4g + 0..3;  p[4], p[5]: rows 16 + 4g + 0..3;  p[6], p[7]: rows 24 + 4g + 0..3
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const auto s0 = __builtin_amdgcn_permlane32_swap(p[e], p[2 + e], false, false);
    p[e] = s0[0];
    p[2 + e] = s0[1];
    const auto s1 = __builtin_amdgcn_permlane32_swap(p[4 + e], p[6 + e], false, false);
    p[4 + e] = s1[0];
    p[6 + e] = s1[1];
  }
  lo = u32x4{p[0], p[1], p[2], p[3]};
  hi = u32x4{p[4], p[5], p[6], p[7]};
}

// The same exchange on fp32 values (two 16-byte chunks of 4 rows each per half): lane (n, g) ends with rows
// 8g .. 8g + 7 and 16 + 8g .. 16 + 8g + 7 of column n in out[0..15] (row order).
__device__ __forceinline__ void rt_regroup_f32(const f32x16& acc, float (&out)[16]) {
  uint32_t p[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) p[e] = __float_as_uint(acc[e]);
  // p[0..3]: rows 4g + 0..3;  p[4..7]: 8 + 4g;  p[8..11]: 16 + 4g;  p[12..15]: 24 + 4g
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const auto s0 = __builtin_amdgcn_permlane32_swap(p[e], p[4 + e], false, false);
    p[e] = s0[0];
    p[4 + e] = s0[1];
    const auto s1 = __builtin_amdgcn_permlane32_swap(p[8 + e], p[12 + e], false, false);
    p[8 + e] = s1[0];
    p[12 + e] = s1[1];
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) out[e] = __uint_as_float(p[e]);
}

// One 16-byte global -> LDS transfer per lane (global_load_lds_dwordx4): the wave's 64 chunks land at lds_base + 16 * lane.
// Issued through inline assembly so that the only waits on it are the explicit s_waitcnt vmcnt of the slab ring (the
// compiler would otherwise drain every outstanding transfer before each LDS read it cannot prove disjoint).  lds_base is
// wave-uniform (it goes through M0).  On this GPU family an LDS DMA that reads M0 right after a scalar write of M0 needs
// one wait state (the s_nop): the compiler's hazard pass does not look inside inline assembly.
__device__ __forceinline__ void lds_dma16(const void* gptr, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(lds_base) : "memory");
}
// The lane index, computed where it is called (volatile: never hoisted, so values derived from it are not kept live
// across a loop in registers the loop needs)
__device__ __forceinline__ int opaque_lane() {
  uint32_t lane;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane));
  return (int)lane;
}

// The same transfer from a wave-uniform base plus a 32-bit per-lane byte offset (scalar base: no 64-bit address per lane).
__device__ __forceinline__ void lds_dma16_s(uint32_t voff, const void* sbase, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds_base) : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p);
}

// Orders a wave's own LDS writes before its later LDS reads of other lanes' data (the LDS unit executes a wave's
// operations in order; this keeps the compiler from moving the reads above the writes).
__device__ __forceinline__ void rt_wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---------------------------------------------------------------------------------------------------------------- fp32 row tiles
// The exact tier's form of the 32-pixel tile on the fp32 matrix core (v_mfma_f32_32x32x2_f32: fp32 operands, products and
// sums).  Lane (n, g) holds pixel n's channels 64 g .. 64 g + 63, and k-step s pairs channel s (g = 0) with 64 + s (g = 1),
// so one 16-byte LDS read gives a lane the weights of 4 consecutive k-steps.  D = W x^T: lane (n, g) holds pixel n and the
// 16 output rows c_row(v, g) = 8 (v / 4) + 4 g + v % 4 of a 32-row block, as in the bf16 form.
constexpr int RTF_WP = RT_C + 4;     // LDS pitch (floats) of a 128-wide fp32 weight row: 16 consecutive rows on distinct banks

__device__ __forceinline__ f32x16 mfma32f(float a, float b, const f32x16& c) { return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0); }

// LayerNorm of the lane's half of a 128-channel fp32 pixel row (row = the pixel's channel 0; zeros when !live): two-pass
// statistics over both halves (exchanged with lane n ^ 32), then the affine (either pointer may be NULL; 16-byte aligned).
// rtf_norm: the same on values already in registers.
__device__ __forceinline__ void rtf_norm(int g, const float* __restrict__ w, const float* __restrict__ b, float eps, float (&xn)[64]) {
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 64; ++k) s += xn[k];
  s += __shfl_xor(s, 32);
  const float mean = s / (float)RT_C;
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < 64; ++k) {
    const float d = xn[k] - mean;
    q += d * d;
  }
  q += __shfl_xor(q, 32);
  const float rstd = 1.0f / sqrtf(q / (float)RT_C + eps);
#pragma unroll
  for (int k = 0; k < 64; ++k) xn[k] = (xn[k] - mean) * rstd;
  if (w) {
#pragma unroll
    for (int s4 = 0; s4 < 16; ++s4) {
      const f32x4 wv = *reinterpret_cast<const f32x4*>(w + 64 * g + 4 * s4);
#pragma unroll
      for (int e = 0; e < 4; ++e) xn[4 * s4 + e] *= wv[e];
    }
  }
  if (b) {
#pragma unroll
    for (int s4 = 0; s4 < 16; ++s4) {
      const f32x4 bv = *reinterpret_cast<const f32x4*>(b + 64 * g + 4 * s4);
#pragma unroll
      for (int e = 0; e < 4; ++e) xn[4 * s4 + e] += bv[e];
    }
  }
}
__device__ __forceinline__ void rtf_ln(const float* row, bool live, int g, const float* __restrict__ w, const float* __restrict__ b,
                                       float eps, float (&xn)[64]) {
#pragma unroll
  for (int s4 = 0; s4 < 16; ++s4) {
    const f32x4 v = live ? *reinterpret_cast<const f32x4*>(row + 64 * g + 4 * s4) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 4; ++e) xn[4 * s4 + e] = v[e];
  }
  rtf_norm(g, w, b, eps, xn);
}

// acc[m] += W_m x^T over 128 channels for K weight blocks of 32 rows held in LDS (w[m] = &block_m[n * RTF_WP + 64 g]), the
// K accumulation chains interleaved, one 4-step group of fragment lookahead.
template <int K>
__device__ __forceinline__ void rtf_gemm(const float* const (&w)[K], const float (&xn)[64], f32x16 (&acc)[K]) {
  f32x4 f[K];
#pragma unroll
  for (int m = 0; m < K; ++m) f[m] = *reinterpret_cast<const f32x4*>(w[m]);
#pragma unroll
  for (int s4 = 0; s4 < 16; ++s4) {
    f32x4 c[K];
#pragma unroll
    for (int m = 0; m < K; ++m) {
      c[m] = f[m];
      if (s4 + 1 < 16) f[m] = *reinterpret_cast<const f32x4*>(w[m] + 4 * s4 + 4);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int m = 0; m < K; ++m) acc[m] = mfma32f(c[m][e], xn[4 * s4 + e], acc[m]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Rows r0 .. r0 + 31 of a [rows][128] fp32 matrix (16-byte aligned) into LDS at pitch RTF_WP, through registers: rtf_fetch
// issues the global loads (NT threads, 1024 / NT float4 each), rtf_put stores them.
template <int NT>
__device__ __forceinline__ void rtf_fetch(const float* __restrict__ m, int64_t r0, int tid, f32x4 (&st)[1024 / NT]) {
#pragma unroll
  for (int q = 0; q < 1024 / NT; ++q) {
    const int i = tid + NT * q;
    st[q] = *reinterpret_cast<const f32x4*>(m + (r0 + (i >> 5)) * RT_C + (i & 31) * 4);
  }
}
template <int NT>
__device__ __forceinline__ void rtf_put(float* lds, int tid, const f32x4 (&st)[1024 / NT]) {
#pragma unroll
  for (int q = 0; q < 1024 / NT; ++q) {
    const int i = tid + NT * q;
    *reinterpret_cast<f32x4*>(lds + (i >> 5) * RTF_WP + (i & 31) * 4) = st[q];
  }
}

}  // namespace fpf
