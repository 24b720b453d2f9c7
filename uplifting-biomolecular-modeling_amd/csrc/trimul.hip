// Triangle multiplication (outgoing / incoming), three launches on the caller's stream:
//   K1        LN_in(z) -> four gated projections -> mask -> channel planes A[c][P][Q], B[c][P][Q] (bf16, tiled: see tl_off)
//             outgoing: plane (P, Q) = z pixel (P, Q);  incoming: plane (P, Q) = z pixel (Q, P) (the transposed load: a wave's
//             32 plane columns are 32 z rows of one column, each a contiguous 256-byte pixel row)
//   contract  X[c][i][j] = sum_k A[c][i][k] B[c][j][k] -- a batched "NT" bf16 MFMA GEMM, fp32 accumulation, bf16 X
//   K3        LN_out(X) W_o^T * sigmoid(LN_in(z) W_og^T) [+ z] -> out (LN_in recomputed from z instead of storing the gate)
// Replaces common/opt_core/opt_core/kernels/trimul/__init__.py:1982 (triangle_multiplication), row `native`'s K1 | bmm | K3
// structure (kernels/trimul/native/DESIGN.md:1-40).  Planes are padded to Np = ceil(N / 128) * 128 with zeros so the
// contraction needs no bounds checks.  The fp32 path (exact tier) has the same three launches in fp32 scalar FMA.
#include <algorithm>

#include <mutex>

#include "rowtile.h"

namespace fpf {

constexpr int TM_C = 128;            // c_z = c_h for the bf16 path
constexpr int TM_TILE = 128;         // contraction tile and plane padding

// Tiled plane layout of the bf16 path: element (b, c, P, Q) of a [B, 128, Np, Np] plane set lives at
// ((b (Np / 32) + Q / 32) Np + P) 4096 + 32 c + Q % 32 -- for each plane row P and 32-column block, the 128 channels' 32
// values form one contiguous 8 KB block, and the blocks of one column block follow each other row by row.  K1 writes a
// 32-pixel tile as whole blocks and K3 reads one as 1 KB-contiguous loads; the contraction reads 64-byte runs of k along
// rows 8 KB apart (TL_ROW) and steps one column block (TL_KBLK(Np)) per 32-wide k slab.
// A plane of Rp rows (the rows mode's slices: Rp < Np rows, all Np columns) has the same layout with Rp rows per column
// block: ((b (Np / 32) + Q / 32) Rp + P) 4096 + 32 c + Q % 32.  The channels mode's operand planes hold a block of cpl
// channels (cpl a multiple of 32) in the same order: ((b (Np / 32) + Q / 32) Rp + P) 32 cpl + 32 c + Q % 32.
constexpr int64_t TL_ROW = 4096;
__device__ __forceinline__ int64_t tl_kblk(int64_t Rp) { return Rp * 4096; }
__host__ __device__ __forceinline__ int64_t tl_off_rc(int64_t b, int64_t c, int64_t P, int64_t Q, int64_t Np, int64_t Rp, int64_t cpl) {
  return ((b * (Np >> 5) + (Q >> 5)) * Rp + P) * (32 * cpl) + c * 32 + (Q & 31);
}
__host__ __device__ __forceinline__ int64_t tl_off_r(int64_t b, int64_t c, int64_t P, int64_t Q, int64_t Np, int64_t Rp) {
  return tl_off_rc(b, c, P, Q, Np, Rp, TM_C);
}
__device__ __forceinline__ int64_t tl_off(int64_t b, int64_t c, int64_t P, int64_t Q, int64_t Np) { return tl_off_r(b, c, P, Q, Np, Np); }

// ---------------------------------------------------------------------------------------------------------------- K1 (bf16)
// Persistent: the four [128 x 128] projection weights live in LDS (139 KB) for the workgroup's lifetime; each wave walks
// 32-column plane tiles (plane row P, columns Q0 .. Q0+31), prefetching the next tile's 32 z rows while it computes.
// NT: planes larger than the 256 MiB last-level cache (2 x 151 MB at N = 768) are written with non-temporal stores, so they
// do not displace z, which K3 reads again (trimul 10-20 us faster per direction at N = 768, the same bits); smaller planes
// stay cacheable for the contraction (non-temporal at N = 512 made it 10-15 us slower).
// ZF32: z is fp32 (the fp32-resident form); each tile's rows are read and rounded to bf16 at the start of its iteration.
// NCB: the 32-channel blocks computed (4: the whole op; fewer: one block of the channels mode, from channel 32 cb0).
template <bool ZF32, int NCB, bool NT>
__global__ void __launch_bounds__(512) trimul_k1_bf16(const void* __restrict__ z, const float* __restrict__ mask,
                                                      const float* __restrict__ ln_w, const float* __restrict__ ln_b, float eps,
                                                      const uint16_t* __restrict__ w_ap, const uint16_t* __restrict__ w_ag,
                                                      const uint16_t* __restrict__ w_bp, const uint16_t* __restrict__ w_bg,
                                                      uint16_t* __restrict__ pa, uint16_t* __restrict__ pb, int64_t N, int64_t Np, int64_t B,
                                                      int outgoing, int cb0) {
  __shared__ __attribute__((aligned(16))) uint16_t sW[4 * RT_C * RT_LD];
  __shared__ __attribute__((aligned(16))) float sLN[2 * RT_C];
  __shared__ __attribute__((aligned(16))) float sM[RT_WAVES][32];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, n = l & 31, g = l >> 5;
  rt_stage_affine(sLN, ln_w, ln_b, tid, 512);
  rt_stage_weights(sW, w_ap, RT_C, RT_C, tid, 512);
  rt_stage_weights(sW + 1 * RT_C * RT_LD, w_ag, RT_C, RT_C, tid, 512);
  rt_stage_weights(sW + 2 * RT_C * RT_LD, w_bp, RT_C, RT_C, tid, 512);
  rt_stage_weights(sW + 3 * RT_C * RT_LD, w_bg, RT_C, RT_C, tid, 512);
  __syncthreads();
  const uint32_t tpr = (uint32_t)(Np / 32), per_b = (uint32_t)Np * tpr, total = (uint32_t)B * per_b;
  const uint32_t stride = gridDim.x * RT_WAVES;
  uint32_t t = blockIdx.x * RT_WAVES + wave;
  u32x4 raw[8];
  auto put = [&](uint16_t* dst, const u32x4& lo, const u32x4& hi) {   // 16 + 16 channel values of one plane row block
    if constexpr (NT) {
      __builtin_nontemporal_store(lo, reinterpret_cast<u32x4*>(dst));
      __builtin_nontemporal_store(hi, reinterpret_cast<u32x4*>(dst + 16));
    } else {
      *reinterpret_cast<u32x4*>(dst) = lo;
      *reinterpret_cast<u32x4*>(dst + 16) = hi;
    }
  };
  auto fetch = [&](uint32_t tt) {
    const RtTile tl = rt_tile(tt, per_b, tpr);
    const int64_t b = tl.b, P = tl.r, Q = tl.c * 32 + n;
    const bool live = P < N && Q < N;
    const int64_t pix = (b * N + (outgoing ? P : Q)) * N + (outgoing ? Q : P);
    if constexpr (ZF32) rt_load_f32(static_cast<const float*>(z) + (live ? pix : 0) * RT_C, live, g, raw);
    else rt_load(static_cast<const uint16_t*>(z) + (live ? pix : 0) * RT_C, live, g, raw);
  };
  if (!ZF32 && t < total) fetch(t);
  for (; t < total; t += stride) {
    if constexpr (ZF32) fetch(t);
    const RtTile tl = rt_tile(t, per_b, tpr);
    const int64_t b = tl.b, P = tl.r, Q = tl.c * 32 + n;
    const bool live = P < N && Q < N;
    const int64_t pix = (b * N + (outgoing ? P : Q)) * N + (outgoing ? Q : P);
    const int64_t Q0 = Q - n, cpl = 32 * NCB;
    uint16_t* oa = pa + tl_off_rc(b, 0, P, Q0, Np, Np, cpl) + 8 * g;
    uint16_t* ob = pb + tl_off_rc(b, 0, P, Q0, Np, Np, cpl) + 8 * g;
    if (P >= N || Q0 >= N) {             // wave-uniform: a tile of plane padding only, whose products are zero
      if (!ZF32 && t + stride < total) fetch(t + stride);
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        const int64_t c = cb * 32 + n;
        const u32x4 zero = {0, 0, 0, 0};
        put(oa + c * 32, zero, zero);
        put(ob + c * 32, zero, zero);
      }
      continue;
    }
    const float m = live ? (mask ? mask[pix] : 1.0f) : 0.0f;
    const bool ones = __builtin_amdgcn_ballot_w64(m != 1.0f) == 0;   // every pixel of the tile kept: no mask products
    bf16x8 xb[8];
    rt_ln(raw, g, sLN, eps, xb);
    if (!ZF32 && t + stride < total) fetch(t + stride);
    // the swapped products put the channel on the lanes and 16 pixels of the tile in the registers: the pixel masks come back
    // from LDS in that order (pixels c_row(v, g) = four runs of 4), and after the lane exchange each lane stores two runs of 8
    // consecutive plane columns
    if (g == 0) sM[wave][n] = m;
    rt_wave_lds_sync();
    float mv[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4 m4 = *reinterpret_cast<const f32x4*>(&sM[wave][8 * q + 4 * g]);
#pragma unroll
      for (int e = 0; e < 4; ++e) mv[4 * q + e] = m4[e];
    }
    rt_wave_lds_sync();
    // channel blocks cb0 .. cb0 + NCB - 1 (32 channels each) into planes of 32 NCB channels (the whole op: 0 .. 3 into 128)
#pragma unroll 1
    for (int cb = 0; cb < NCB; ++cb) {
      const uint16_t* const ws[4] = {sW, sW + 1 * RT_C * RT_LD, sW + 2 * RT_C * RT_LD, sW + 3 * RT_C * RT_LD};
      f32x16 acc[4];
      rt_gemm32_multi_xw<4>(ws, (cb0 + cb) * 32, n, g, xb, acc);
      f32x16 va, vb;
      if (ones) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          va[v] = sigmoidf_(acc[1][v]) * acc[0][v];
          vb[v] = sigmoidf_(acc[3][v]) * acc[2][v];
        }
      } else {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          va[v] = mv[v] * sigmoidf_(acc[1][v]) * acc[0][v];
          vb[v] = mv[v] * sigmoidf_(acc[3][v]) * acc[2][v];
        }
      }
      const int64_t c = cb * 32 + n;
      u32x4 lo, hi;
      rt_pack16(va, lo, hi);
      put(oa + c * 32, lo, hi);
      rt_pack16(vb, lo, hi);
      put(ob + c * 32, lo, hi);
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------- contraction, 256 x 256 tiles
// Planes padded to a multiple of 128: a workgroup (4 waves, one per SIMD) computes 256 x 256 tiles of X, each wave a 128 x 128
// quarter in 16 accumulators.  Where the rows (or columns) end 128 into a tile (a padded extent of an odd multiple of 128),
// that tile's upper 128 rows of the operand re-read its lower 128 (the DMA addresses of slots 512 .. 1023 step back 128 rows),
// so nothing is read past the plane; the duplicated quarters are computed and not stored.  The grid is persistent (one workgroup per CU): workgroup b runs on XCD b % 8
// (round-robin dispatch), XCD x owns the contiguous tile range [x per, (x + 1) per) and its workgroups take every
// (grid / 8)-th tile of it, so the tiles that share A rows / B rows of one plane are computed by one XCD at the same time.
// The A and B k-slabs (256 rows x 32 k each) go straight from global memory into LDS (global_load_lds_dwordx4: no VGPR
// staging) through a ring of CB_NBUF buffers with CB_IF slabs in flight; the slab stream runs across tile boundaries, so
// the next tile's first slabs land while the current tile finishes and its stores drain behind the next tile's MFMAs.
// Within a slab row the four 16-byte chunks are XOR-swizzled by (row >> 2) & 3, so the fragment reads of 16 consecutive
// rows land on 16 distinct bank groups.  The MFMA runs with the operands exchanged (D = B A^T): lane = row i, registers =
// 16 columns j, and after the half-wave lane exchange each lane stores 8 consecutive columns per 16-byte store.
constexpr int CB_T = 256, CB_K = 32, CB_NBUF = 4, CB_IF = CB_NBUF - 1;

// waits until at most p slabs (8 transfers of this wave each) are outstanding, plus the 32 stores of the previous tile when
// they were issued after the awaited slab (the vector-memory counter retires loads and stores in issue order)
__device__ __forceinline__ void cb_wait(int p, bool stores) {
  static_assert(CB_IF <= 4, "the waits below count at most 4 slabs in flight");
  if (stores) {
    if (p >= 3) asm volatile("s_waitcnt vmcnt(56)" ::: "memory");
    else if (p == 2) asm volatile("s_waitcnt vmcnt(48)" ::: "memory");
    else if (p == 1) asm volatile("s_waitcnt vmcnt(40)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(32)" ::: "memory");
  } else {
    if (p >= 3) asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
    else if (p == 2) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    else if (p == 1) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
}

// CPL: the channels the operand planes hold (128: the whole op; 32 / 64: one block of the channels mode, whose channel c is
// channel cx0 + c of X).
template <int CPL>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
trimul_contract_bf16_256(const uint16_t* __restrict__ A, const uint16_t* __restrict__ Bm, uint16_t* __restrict__ X, int64_t Np, int64_t Nk,
                         int64_t nbatch, int64_t La, int64_t a0, int64_t Ra, int cx0) {
  constexpr int64_t cpl = CPL;
  __shared__ __attribute__((aligned(16))) uint16_t sA[CB_NBUF][CB_T * CB_K];
  __shared__ __attribute__((aligned(16))) uint16_t sB[CB_NBUF][CB_T * CB_K];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, n = l & 31, g = l >> 5;
  const int64_t tpd = cdiv(Np, CB_T), tiles = cdiv(Ra, CB_T) * tpd, total = tiles * nbatch;   // A rows a0 .. a0 + Ra - 1, B whole
  const int64_t per = (total + 7) / 8, g8 = gridDim.x / 8;     // the host launches a multiple of 8 workgroups
  const int64_t x0 = (blockIdx.x % 8) * per, first = x0 + blockIdx.x / 8, end = total < x0 + per ? total : x0 + per;
  if (first >= end) return;
  const int ntile = (int)((end - first + g8 - 1) / g8);       // tiles first, first + g8, ... below end
  const int nk = (int)(Nk / CB_K), U = ntile * nk;             // slabs per tile, slabs of this workgroup (host: U < 2^31)
  // the operand planes hold cpl channels (128: the whole op; the channels mode's block otherwise), batch index bc = b cpl + c;
  // X holds all 128, this call's channel c at cx0 + c
  constexpr int64_t orow = 32 * cpl;
  const int64_t kstride_a = La * orow, kstride_b = Np * orow;
  auto tile_of = [&](int r, int64_t& bc, int64_t& ti, int64_t& tj) {
    const int64_t w = first + (int64_t)r * g8, t = w % tiles;
    bc = w / tiles;
    ti = t / tpd;
    tj = t % tpd;
  };
  // slab loads: 1024 16-byte chunks per operand; instruction q of thread tid fills LDS slot s = 256 q + tid (each wave
  // instruction writes 1 KB contiguously); slot s = row s >> 2, position s & 3, holding chunk (s & 3) ^ ((row >> 2) & 3)
  uint32_t goff[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int sl = 256 * q + tid, r = sl >> 2, c = (sl & 3) ^ ((r >> 2) & 3);
    goff[q] = (uint32_t)(r * orow + 8 * c);
  }
  // issue cursor: the next slab to load is slab ikt of tile ir (operand bases ia0 / ib0 of slots 0 .. 511, rows 0 .. 127 of the
  // tile; ia1 / ib1 of slots 512 .. 1023, rows 128 .. 255, or rows 0 .. 127 again where the tile is half inside)
  int ir = 0, ikt = 0;
  const uint16_t *ia0, *ib0, *ia1, *ib1;
  auto set_bases = [&](int r) {
    int64_t bc, ti, tj;
    tile_of(r, bc, ti, tj);
    ia0 = A + tl_off_rc(bc / cpl, bc % cpl, a0 + ti * CB_T, 0, Np, La, cpl);
    ib0 = Bm + tl_off_rc(bc / cpl, bc % cpl, tj * CB_T, 0, Np, Np, cpl);
    ia1 = ti * CB_T + CB_T > Ra ? ia0 - 128 * orow : ia0;
    ib1 = tj * CB_T + CB_T > Np ? ib0 - 128 * orow : ib0;
  };
  set_bases(0);
  auto issue_next = [&](int buf) {
    const int64_t koa = (int64_t)ikt * kstride_a, kob = (int64_t)ikt * kstride_b;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      lds_dma16((q < 2 ? ia0 : ia1) + goff[q] + koa, lds_addr(&sA[buf][(256 * q + 64 * wave) * 8]));
      lds_dma16((q < 2 ? ib0 : ib1) + goff[q] + kob, lds_addr(&sB[buf][(256 * q + 64 * wave) * 8]));
    }
    if (++ikt == nk) {
      ikt = 0;
      if (++ir < ntile) set_bases(ir);
    }
  };
  const int wr = (wave >> 1) * 128, wc = (wave & 1) * 128;
  // fragment read offsets (elements) of this lane's rows for chunk position 0 / 1 of each k16 half: row r, chunk c
  auto frag_off = [&](int r, int c) { return (r * 4 + (c ^ ((r >> 2) & 3))) * 8; };
  f32x16 acc[4][4];
  // the 16 fragments of one slab: A rows wr + 32 s + n, B rows wc + 32 s + n, chunks 2 ks + g
  auto read_frags = [&](int buf, bf16x8 (&fa)[2][4], bf16x8 (&fb)[2][4]) {
    const uint16_t* pa = sA[buf];
    const uint16_t* pb = sB[buf];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        fa[ks][s4] = as_bf8(*reinterpret_cast<const u32x4*>(pa + frag_off(wr + 32 * s4 + n, 2 * ks + g)));
        fb[ks][s4] = as_bf8(*reinterpret_cast<const u32x4*>(pb + frag_off(wc + 32 * s4 + n, 2 * ks + g)));
      }
  };
  // ring: slab u lives in buffer u % CB_NBUF, CB_IF slabs in flight.  Slab u issues slab u + CB_IF (its buffer held slab
  // u - 1, whose fragments every wave read before slab u - 1's barrier), runs 8 of its 32 MFMAs, waits for slab u + 1 at
  // the barrier (the matrix core keeps working), then reads slab u + 1's 16 fragments ahead of the other 24 MFMAs.  A
  // tile's stores are issued after the DMA of the next tile's slabs 0 .. CB_IF - 1 and before that of slab CB_IF, so the
  // waits for slabs 1 .. CB_IF - 1 of the next tile count them -- in the waves that stored (a wave whose quarter of a
  // half-inside tile is a duplicate issues none, and counting stores it never issued would end its wait early).
  for (int s = 0; s < CB_IF && s < U; ++s) issue_next(s);
  cb_wait((U < CB_IF ? U : CB_IF) - 1, false);
  __builtin_amdgcn_s_barrier();
  // two fragment sets that trade roles every slab (no register copies between slabs: a copy into registers the queued
  // MFMAs still read would hold the wave until those MFMAs start)
  bf16x8 f0a[2][4], f0b[2][4], f1a[2][4], f1b[2][4];
  read_frags(0, f0a, f0b);
  // ring buffers of the next slab to issue (slab u + CB_IF) and of the next slab to read (u + 1), stepped once per slab
  int bi = CB_IF % CB_NBUF, br = 1 % CB_NBUF;
  auto slab = [&](bool stores, int u, const bf16x8 (&fa)[2][4], const bf16x8 (&fb)[2][4], bf16x8 (&na)[2][4], bf16x8 (&nb)[2][4]) {
    if (u + CB_IF < U) issue_next(bi);
    bi = bi == CB_NBUF - 1 ? 0 : bi + 1;
#pragma unroll
    for (int si = 0; si < 4; ++si)
#pragma unroll
      for (int sj = 0; sj < 2; ++sj) acc[si][sj] = mfma32(fb[0][sj], fa[0][si], acc[si][sj]);
    __builtin_amdgcn_sched_barrier(0);
    if (u + 1 < U) {                                     // slab u + 1 landed
      cb_wait(U - 2 - u < CB_IF - 1 ? U - 2 - u : CB_IF - 1, stores);
      __builtin_amdgcn_s_barrier();
    }
    __builtin_amdgcn_sched_barrier(0);
    if (u + 1 < U) read_frags(br, na, nb);
    br = br == CB_NBUF - 1 ? 0 : br + 1;
#pragma unroll
    for (int si = 0; si < 4; ++si)
#pragma unroll
      for (int sj = 2; sj < 4; ++sj) acc[si][sj] = mfma32(fb[0][sj], fa[0][si], acc[si][sj]);
#pragma unroll
    for (int si = 0; si < 4; ++si)
#pragma unroll
      for (int sj = 0; sj < 4; ++sj) acc[si][sj] = mfma32(fb[1][sj], fa[1][si], acc[si][sj]);
    __builtin_amdgcn_sched_barrier(0);
  };
  bool stored = false;                                   // this wave issued the previous tile's 32 stores
  for (int r = 0; r < ntile; ++r) {
#pragma unroll
    for (int si = 0; si < 4; ++si)
#pragma unroll
      for (int sj = 0; sj < 4; ++sj) acc[si][sj] = f32x16{};
    const int u0 = r * nk;
    // the previous tile's stores were issued after this tile's slabs 0 .. CB_IF - 1: the waits for slabs 1 .. CB_IF - 1 (in slabs
    // 0 .. CB_IF - 2) count them
    slab(stored, u0, f0a, f0b, f1a, f1b);                // nk is even: Nk is a multiple of 64
    slab(stored, u0 + 1, f1a, f1b, f0a, f0b);
    for (int kt = 2; kt < nk; kt += 2) {
      slab(stored && kt <= CB_IF - 2, u0 + kt, f0a, f0b, f1a, f1b);
      slab(stored && kt + 1 <= CB_IF - 2, u0 + kt + 1, f1a, f1b, f0a, f0b);
    }
    int64_t bc, ti, tj;
    tile_of(r, bc, ti, tj);
    const int64_t pb_ = bc / cpl, pc = cx0 + bc % cpl;
    // the lane's part of the store offsets, recomputed per tile (kept live across the slab loop it would take registers
    // the loop needs): row n of each 32-row block, 8 g columns in
    const uint32_t lane = (uint32_t)opaque_lane();
    const uint32_t lane_el = (lane & 31) * (uint32_t)TL_ROW + 8 * (lane >> 5);
    // a quarter past the rows (or columns) of a half-inside tile holds duplicates: not stored (a wave-uniform branch around the
    // whole store sequence, so the accumulators are still packed and stored one at a time)
    stored = ti * CB_T + wr < Ra && tj * CB_T + wc < Np;
    if (stored) {
#pragma unroll
      for (int si = 0; si < 4; ++si)
#pragma unroll
        for (int sj = 0; sj < 4; ++sj) {
          u32x4 lo, hi;
          rt_pack16(acc[si][sj], lo, hi);
          uint16_t* xp = X + tl_off_r(pb_, pc, ti * CB_T + wr + 32 * si, tj * CB_T + wc + 32 * sj, Np, Ra) + lane_el;
          *reinterpret_cast<u32x4*>(xp) = lo;
          *reinterpret_cast<u32x4*>(xp + 16) = hi;
          __builtin_amdgcn_sched_barrier(0);             // one accumulator at a time (bounded VGPR use)
        }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------- K3 (bf16)
// Output rows i0 .. i0 + rows - 1 (the whole op: 0 .. N - 1), X read from a plane of Rx rows whose row 0 is plane row x0.
// Persistent: W_o and W_og live in LDS (70 KB; with the per-wave X slots one workgroup of 8 waves per CU, so registers up
// to 256 cost no occupancy).  Each wave scatters its X tile X[c][i][j0 .. j0+31] (channel-major, 128 rows of 64 B, loaded
// during the previous tile) pixel-major into a private LDS slot, so the LN_out / B-operand reads are 16-byte rows, issues
// the next tile's X loads, then LN_out(X) W_o^T * sigmoid(LN_in(z) W_og^T) [+ z] (the residual reuses the z rows the
// LayerNorm read).
constexpr int K3_XLD = RT_C + 8;     // LDS pitch of the staged X tile, pixel-major [32 pixels][128 channels]
// Channel c of pixel p sits at column c ^ k3_swz(p): the 2-byte scatter writes pixels p0 + 2e, p0 = 0, 8, 16, 24, in one
// instruction, rows that any 16-byte-aligned pitch puts on the same banks; the XOR moves them 0 / 8 / 16 / 24 dwords apart,
// and every 8-channel chunk stays contiguous for the 16-byte fragment reads
__device__ __forceinline__ int k3_swz(int p) { return 16 * ((p >> 3) & 3); }

// ZF32: z and out are fp32 (the fp32-resident form): LN_in reads the bf16 copy of each row, the residual adds the fp32 z
// and the result is stored in fp32.
template <bool ZF32>
__global__ void __launch_bounds__(512) trimul_k3_bf16(const void* zin, void* out, const uint16_t* __restrict__ X,
                                                      const float* __restrict__ ln_in_w, const float* __restrict__ ln_in_b,
                                                      const float* __restrict__ ln_out_w, const float* __restrict__ ln_out_b, float eps,
                                                      const uint16_t* __restrict__ w_o, const uint16_t* __restrict__ w_og,
                                                      int64_t N, int64_t Np, int64_t B, int residual, int64_t i0, int64_t rows, int64_t x0, int64_t Rx) {
  __shared__ __attribute__((aligned(16))) uint16_t sW[2 * RT_C * RT_LD];
  __shared__ __attribute__((aligned(16))) uint16_t sX[RT_WAVES][32 * K3_XLD];
  __shared__ __attribute__((aligned(16))) float sLNo[2 * RT_C];
  __shared__ __attribute__((aligned(16))) float sLNi[2 * RT_C];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, n = l & 31, g = l >> 5;
  rt_stage_affine(sLNo, ln_out_w, ln_out_b, tid, 512);
  rt_stage_affine(sLNi, ln_in_w, ln_in_b, tid, 512);
  rt_stage_weights(sW, w_o, RT_C, RT_C, tid, 512);
  rt_stage_weights(sW + RT_C * RT_LD, w_og, RT_C, RT_C, tid, 512);
  __syncthreads();
  const uint32_t tpr = (uint32_t)cdiv(N, 32), per_b = (uint32_t)rows * tpr, total = (uint32_t)B * per_b;
  const uint32_t stride = gridDim.x * RT_WAVES;
  uint16_t* sx = sX[wave];
  uint32_t t = blockIdx.x * RT_WAVES + wave;
  u32x4 rx[8], rz[8];
  auto fetch_x = [&](uint32_t tt) {                       // the tile's 8 KB X block (rows padded to Np: in bounds)
    const RtTile tl = rt_tile(tt, per_b, tpr);
    const uint16_t* xs = X + tl_off_r(tl.b, 0, i0 + tl.r - x0, tl.c * 32, Np, Rx);
#pragma unroll
    for (int it = 0; it < 8; ++it) rx[it] = *reinterpret_cast<const u32x4*>(xs + 8 * (l + 64 * it));   // channel q >> 2, chunk q & 3
  };
  if (t < total) fetch_x(t);
  for (; t < total; t += stride) {
    const RtTile tl = rt_tile(t, per_b, tpr);
    const int64_t b = tl.b, i = i0 + tl.r, j = tl.c * 32 + n;
    const bool live = j < N;
    const int64_t pix = (b * N + i) * N + j;
    if constexpr (ZF32) rt_load_f32(static_cast<const float*>(zin) + ((b * N + i) * N + (live ? j : 0)) * RT_C, live, g, rz);
    else rt_load(static_cast<const uint16_t*>(zin) + ((b * N + i) * N + (live ? j : 0)) * RT_C, live, g, rz);
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int q = l + 64 * it, c = q >> 2, p0 = (q & 3) * 8;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sx[(p0 + 2 * e) * K3_XLD + (c ^ k3_swz(p0 + 2 * e))] = (uint16_t)(rx[it][e] & 0xffff);
        sx[(p0 + 2 * e + 1) * K3_XLD + (c ^ k3_swz(p0 + 2 * e + 1))] = (uint16_t)(rx[it][e] >> 16);
      }
    }
    rt_wave_lds_sync();
    if (t + stride < total) fetch_x(t + stride);            // the next tile's X lands while this one computes
    u32x4 xr[8];
#pragma unroll
    for (int tt = 0; tt < 8; ++tt) xr[tt] = *reinterpret_cast<const u32x4*>(&sx[n * K3_XLD + ((8 * rt_chunk(tt, g)) ^ k3_swz(n))]);
    rt_wave_lds_sync();
    bf16x8 xo[8], xi[8];
    rt_ln(xr, g, sLNo, eps, xo);
    __builtin_amdgcn_sched_barrier(0);      // one LayerNorm's temporaries at a time
    rt_ln(rz, g, sLNi, eps, xi);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      const f32x16 o = rt_gemm32(sW, cb * 32, n, g, xo);
      const f32x16 gt = rt_gemm32(sW + RT_C * RT_LD, cb * 32, n, g, xi);
      f32x16 u;
#pragma unroll
      for (int v = 0; v < 16; ++v) u[v] = sigmoidf_(gt[v]) * o[v];
      // lane (n, g) ends with channels cb*32 + 8g .. +7 and cb*32 + 16 + 8g .. +7 of pixel n: two 16-byte stores
      float y[16];
      rt_regroup_f32(u, y);
      if (!live) continue;
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const int64_t c0 = pix * RT_C + cb * 32 + 16 * h2 + 8 * g;
        if constexpr (ZF32) {
          float* of = static_cast<float*>(out) + c0;
          if (residual) {
            const float* zf = static_cast<const float*>(zin) + c0;
            const f32x4 r0 = *reinterpret_cast<const f32x4*>(zf), r1 = *reinterpret_cast<const f32x4*>(zf + 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              y[8 * h2 + e] += r0[e];
              y[8 * h2 + 4 + e] += r1[e];
            }
          }
          *reinterpret_cast<f32x4*>(of) = f32x4{y[8 * h2], y[8 * h2 + 1], y[8 * h2 + 2], y[8 * h2 + 3]};
          *reinterpret_cast<f32x4*>(of + 4) = f32x4{y[8 * h2 + 4], y[8 * h2 + 5], y[8 * h2 + 6], y[8 * h2 + 7]};
        } else {
          if (residual) {
            const u32x4 r = rz[2 * cb + h2];                  // z rows chunk 2cb + h2: channels cb*32 + 16 h2 + 8g .. +7
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              y[8 * h2 + 2 * e] += lo_bf(r[e]);
              y[8 * h2 + 2 * e + 1] += hi_bf(r[e]);
            }
          }
          *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + c0) =
              u32x4{pack2(y[8 * h2], y[8 * h2 + 1]), pack2(y[8 * h2 + 2], y[8 * h2 + 3]), pack2(y[8 * h2 + 4], y[8 * h2 + 5]),
                    pack2(y[8 * h2 + 6], y[8 * h2 + 7])};
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------- fp32 path
constexpr int F_R = 32;      // pixel rows per workgroup
constexpr int F_CC = 16;     // output channels per chunk
constexpr int F_CM = 128;    // max channel width

// LayerNorm of 32 rows of fp32 held in LDS (8 threads per row), in place.
__device__ __forceinline__ void ln_rows_lds(float (*xs)[F_CM + 1], int c, const float* w, const float* b, float eps, int tid) {
  const int r = tid >> 3, sub = tid & 7;
  float s = 0.f;
  for (int cc = sub; cc < c; cc += 8) s += xs[r][cc];
  for (int o = 4; o >= 1; o >>= 1) s += __shfl_xor(s, o, 8);
  const float mean = s / (float)c;
  float q = 0.f;
  for (int cc = sub; cc < c; cc += 8) {
    const float d = xs[r][cc] - mean;
    q += d * d;
  }
  for (int o = 4; o >= 1; o >>= 1) q += __shfl_xor(q, o, 8);
  const float rstd = 1.0f / sqrtf(q / (float)c + eps);
  __syncthreads();
  for (int cc = sub; cc < c; cc += 8) xs[r][cc] = (xs[r][cc] - mean) * rstd * (w ? w[cc] : 1.f) + (b ? b[cc] : 0.f);
  __syncthreads();
}

__global__ void __launch_bounds__(256) trimul_k1_f32(const float* __restrict__ z, const float* __restrict__ mask, const float* __restrict__ ln_w,
                                                     const float* __restrict__ ln_b, float eps, const float* __restrict__ w_ap,
                                                     const float* __restrict__ w_ag, const float* __restrict__ w_bp, const float* __restrict__ w_bg,
                                                     float* __restrict__ pa, float* __restrict__ pb, int64_t N, int64_t Np, int cz, int ch, int outgoing) {
  __shared__ float xs[F_R][F_CM + 1];
  __shared__ float ws[4][F_CC][F_CM + 1];
  const int tid = threadIdx.x;
  const int64_t tiles_per_row = Np / F_R;
  const int64_t P = blockIdx.x / tiles_per_row, Q0 = (blockIdx.x % tiles_per_row) * F_R;
  const int64_t b = blockIdx.y;
  for (int i = tid; i < F_R * cz; i += 256) {
    const int r = i / cz, cc = i % cz;
    const int64_t Q = Q0 + r;
    const bool live = P < N && Q < N;
    const int64_t pix = outgoing ? (b * N + P) * N + Q : (b * N + Q) * N + P;
    xs[r][cc] = live ? z[pix * cz + cc] : 0.f;
  }
  __syncthreads();
  ln_rows_lds(xs, cz, ln_w, ln_b, eps, tid);
  const int r = tid >> 3, sub = tid & 7;
  const int64_t Q = Q0 + r;
  const bool live = P < N && Q < N;
  const int64_t pix = outgoing ? (b * N + P) * N + Q : (b * N + Q) * N + P;
  const float m = live ? (mask ? mask[pix] : 1.0f) : 0.0f;
  const int64_t plane = Np * Np;
  for (int c0 = 0; c0 < ch; c0 += F_CC) {
    __syncthreads();
    for (int i = tid; i < F_CC * cz; i += 256) {
      const int j = i / cz, cc = i % cz;
      const bool ok = c0 + j < ch;
      ws[0][j][cc] = ok ? w_ap[(int64_t)(c0 + j) * cz + cc] : 0.f;
      ws[1][j][cc] = ok ? w_ag[(int64_t)(c0 + j) * cz + cc] : 0.f;
      ws[2][j][cc] = ok ? w_bp[(int64_t)(c0 + j) * cz + cc] : 0.f;
      ws[3][j][cc] = ok ? w_bg[(int64_t)(c0 + j) * cz + cc] : 0.f;
    }
    __syncthreads();
    for (int jj = 0; jj < 2; ++jj) {
      const int j = sub * 2 + jj;
      if (c0 + j >= ch) continue;
      float ap = 0.f, ag = 0.f, bp = 0.f, bg = 0.f;
      for (int cc = 0; cc < cz; ++cc) {
        const float xv = xs[r][cc];
        ap = fmaf(xv, ws[0][j][cc], ap);
        ag = fmaf(xv, ws[1][j][cc], ag);
        bp = fmaf(xv, ws[2][j][cc], bp);
        bg = fmaf(xv, ws[3][j][cc], bg);
      }
      const int64_t o = (b * ch + c0 + j) * plane + P * Np + Q;
      pa[o] = m * sigmoid_exact(ag) * ap;
      pb[o] = m * sigmoid_exact(bg) * bp;
    }
  }
}

constexpr int SG_T = 64, SG_K = 16;

__global__ void __launch_bounds__(256) trimul_contract_f32(const float* __restrict__ A, const float* __restrict__ Bm, float* __restrict__ X,
                                                           int64_t Np, int64_t N) {
  __shared__ float sA[SG_K][SG_T + 4];
  __shared__ float sB[SG_K][SG_T + 4];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int64_t bc = blockIdx.z;
  const int64_t i0 = (int64_t)blockIdx.y * SG_T, j0 = (int64_t)blockIdx.x * SG_T;
  const int64_t plane = Np * Np;
  const float* a0 = A + bc * plane;
  const float* b0 = Bm + bc * plane;
  float acc[4][4] = {};
  for (int64_t k0 = 0; k0 < Np; k0 += SG_K) {
    __syncthreads();
    for (int i = tid; i < SG_T * SG_K; i += 256) {
      const int r = i / SG_K, kk = i % SG_K;
      sA[kk][r] = a0[(i0 + r) * Np + k0 + kk];
      sB[kk][r] = b0[(j0 + r) * Np + k0 + kk];
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < SG_K; ++kk) {
      float av[4], bv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        av[u] = sA[kk][ty * 4 + u];
        bv[u] = sB[kk][tx * 4 + u];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int w = 0; w < 4; ++w) acc[u][w] = fmaf(av[u], bv[w], acc[u][w]);
    }
  }
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int64_t i = i0 + ty * 4 + u, j = j0 + tx * 4 + w;
      if (i < N && j < N) X[bc * plane + i * Np + j] = acc[u][w];
    }
}

__global__ void __launch_bounds__(256) trimul_k3_f32(const float* zin, float* out, const float* __restrict__ X, const float* __restrict__ ln_in_w,
                                                     const float* __restrict__ ln_in_b, const float* __restrict__ ln_out_w,
                                                     const float* __restrict__ ln_out_b, float eps, const float* __restrict__ w_o,
                                                     const float* __restrict__ w_og, int64_t N, int64_t Np, int cz, int ch, int residual) {
  __shared__ float xs[F_R][F_CM + 1];
  __shared__ float zs[F_R][F_CM + 1];
  __shared__ float ws[2][F_CC][F_CM + 1];
  const int tid = threadIdx.x;
  const int64_t tiles_per_row = Np / F_R;
  const int64_t i = blockIdx.x / tiles_per_row, j0 = (blockIdx.x % tiles_per_row) * F_R;
  const int64_t b = blockIdx.y;
  const int64_t plane = Np * Np;
  for (int q = tid; q < F_R * ch; q += 256) {
    const int c = q / F_R, r = q % F_R;
    xs[r][c] = (i < N && j0 + r < N) ? X[(b * ch + c) * plane + i * Np + j0 + r] : 0.f;
  }
  for (int q = tid; q < F_R * cz; q += 256) {
    const int r = q / cz, cc = q % cz;
    const int64_t j = j0 + r;
    zs[r][cc] = (i < N && j < N) ? zin[((b * N + i) * N + j) * cz + cc] : 0.f;
  }
  __syncthreads();
  ln_rows_lds(xs, ch, ln_out_w, ln_out_b, eps, tid);
  ln_rows_lds(zs, cz, ln_in_w, ln_in_b, eps, tid);
  const int r = tid >> 3, sub = tid & 7;
  const int64_t j = j0 + r;
  const bool live = i < N && j < N;
  const int64_t pix = (b * N + i) * N + j;
  float y[F_CC / 8 * (F_CM / F_CC)];
  int ny = 0;
  for (int c0 = 0; c0 < cz; c0 += F_CC) {
    __syncthreads();
    for (int q = tid; q < F_CC * F_CM; q += 256) {
      const int jj = q / F_CM, cc = q % F_CM;
      const bool ok = c0 + jj < cz;
      ws[0][jj][cc] = (ok && cc < ch) ? w_o[(int64_t)(c0 + jj) * ch + cc] : 0.f;
      ws[1][jj][cc] = (ok && cc < cz) ? w_og[(int64_t)(c0 + jj) * cz + cc] : 0.f;
    }
    __syncthreads();
    for (int jj = 0; jj < 2; ++jj) {
      const int co = sub * 2 + jj;
      float o = 0.f, gt = 0.f;
      for (int cc = 0; cc < ch; ++cc) o = fmaf(xs[r][cc], ws[0][co][cc], o);
      for (int cc = 0; cc < cz; ++cc) gt = fmaf(zs[r][cc], ws[1][co][cc], gt);
      y[ny++] = sigmoid_exact(gt) * o;
    }
  }
  if (!live) return;
  ny = 0;
  for (int c0 = 0; c0 < cz; c0 += F_CC)
    for (int jj = 0; jj < 2; ++jj) {
      const int co = c0 + sub * 2 + jj;
      float v = y[ny++];
      if (co >= cz) continue;
      if (residual) v += zin[pix * cz + co];
      out[pix * cz + co] = v;
    }
}

// ---------------------------------------------------------------------------------------------------------------- fp32 on the matrix core
// The exact tier at c_z = c_h = 128 (v_mfma_f32_32x32x2_f32: fp32 operands, products and sums), on the fp32 path's
// row-major planes [B 128][Np][Np].  K1 and K3 take one 32-pixel tile per wave (the fp32 row-tile form of rowtile.h), the
// weights of one 32-channel output block at a time in LDS (two buffers, the next block's global loads in flight while the
// current one feeds the MFMAs); the contraction takes 128 x 128 tiles of X per workgroup of 4 waves (64 x 64 each), k in
// slabs of 16 through two LDS buffers.
constexpr int FM_NW = 8;                    // waves per workgroup of K1 / K3
constexpr int FC_T = 128, FC_K = 16, FC_P = FC_K + 4;   // contraction tile, k-slab, LDS pitch (floats) of a slab row

// K1: tile = plane row P, columns Q0 .. Q0 + 31 (pixel (P, Q) outgoing, (Q, P) incoming); every plane element is written,
// padding (P or Q >= N) as 0 (the mask factor of a pixel outside the image is 0).
__global__ void __launch_bounds__(64 * FM_NW) trimul_k1_f32m(const float* __restrict__ z, const float* __restrict__ mask,
                                                             const float* __restrict__ ln_w, const float* __restrict__ ln_b, float eps,
                                                             const float* __restrict__ w_ap, const float* __restrict__ w_ag,
                                                             const float* __restrict__ w_bp, const float* __restrict__ w_bg,
                                                             float* __restrict__ pa, float* __restrict__ pb, int64_t N, int64_t Np, int outgoing) {
  __shared__ __attribute__((aligned(16))) float sW[2][4][32 * RTF_WP];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, n = l & 31, g = l >> 5;
  const int64_t b = blockIdx.y, tpr = Np / 32, tile = (int64_t)blockIdx.x * FM_NW + wave;
  const int64_t P = tile / tpr, Q = (tile % tpr) * 32 + n;
  const bool inb = P < Np;                           // always, for Np a multiple of 128; kept for the stores
  const bool live = inb && P < N && Q < N;
  const int64_t pix = outgoing ? (b * N + P) * N + Q : (b * N + Q) * N + P;
  const float* const W[4] = {w_ap, w_ag, w_bp, w_bg};
  f32x4 st[2][1024 / (64 * FM_NW)];                  // staging of two of the four matrices at a time
  float xn[64];
  rtf_ln(z + (live ? pix : 0) * RT_C, live, g, ln_w, ln_b, eps, xn);
  const float mk = live ? (mask ? mask[pix] : 1.0f) : 0.0f;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int m = 0; m < 2; ++m) rtf_fetch<64 * FM_NW>(W[2 * h + m], 0, tid, st[m]);
#pragma unroll
    for (int m = 0; m < 2; ++m) rtf_put<64 * FM_NW>(sW[0][2 * h + m], tid, st[m]);
  }
  __syncthreads();
  const int64_t plane = Np * Np;
  for (int cb = 0; cb < 4; ++cb) {
    const int buf = cb & 1;
    // block cb + 1 goes to buffer buf ^ 1 (block cb - 1, read by every wave before the last barrier): W_ap / W_ag loads in
    // flight during the MFMAs, W_bp / W_bg during the stores
    if (cb + 1 < 4) {
#pragma unroll
      for (int m = 0; m < 2; ++m) rtf_fetch<64 * FM_NW>(W[m], 32 * (cb + 1), tid, st[m]);
    }
    f32x16 acc[4] = {f32x16{}, f32x16{}, f32x16{}, f32x16{}};
    const float* const w[4] = {&sW[buf][0][n * RTF_WP + 64 * g], &sW[buf][1][n * RTF_WP + 64 * g], &sW[buf][2][n * RTF_WP + 64 * g],
                               &sW[buf][3][n * RTF_WP + 64 * g]};
    rtf_gemm<4>(w, xn, acc);
    if (cb + 1 < 4) {
#pragma unroll
      for (int m = 0; m < 2; ++m) rtf_put<64 * FM_NW>(sW[buf ^ 1][m], tid, st[m]);
#pragma unroll
      for (int m = 0; m < 2; ++m) rtf_fetch<64 * FM_NW>(W[2 + m], 32 * (cb + 1), tid, st[m]);
    }
    if (inb) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t c = 32 * cb + 8 * (v >> 2) + 4 * g + (v & 3);
        const int64_t o = (b * RT_C + c) * plane + P * Np + Q;
        pa[o] = mk * sigmoid_exact(acc[1][v]) * acc[0][v];
        pb[o] = mk * sigmoid_exact(acc[3][v]) * acc[2][v];
      }
    }
    if (cb + 1 < 4) {
#pragma unroll
      for (int m = 0; m < 2; ++m) rtf_put<64 * FM_NW>(sW[buf ^ 1][2 + m], tid, st[m]);
      __syncthreads();
    }
  }
}

// X[bc][i][j] = sum_k A[bc][i][k] B[bc][j][k] for a 128 x 128 tile; X rows / columns at or past N are not written.  k-step s
// of a slab pairs k = s (g = 0) with 8 + s (g = 1), so each lane's 8 slab values of a row are two 16-byte LDS reads.
__global__ void __launch_bounds__(256) trimul_contract_f32m(const float* __restrict__ A, const float* __restrict__ Bm, float* __restrict__ X,
                                                            int64_t Np, int64_t N) {
  __shared__ __attribute__((aligned(16))) float sA[2][FC_T * FC_P];
  __shared__ __attribute__((aligned(16))) float sB[2][FC_T * FC_P];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, n = l & 31, g = l >> 5;
  const int64_t bc = blockIdx.z, plane = Np * Np;
  const float* a0 = A + bc * plane + (int64_t)blockIdx.y * FC_T * Np;
  const float* b0 = Bm + bc * plane + (int64_t)blockIdx.x * FC_T * Np;
  const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
  f32x4 sta[2], stb[2];
  auto fetch = [&](int64_t k0) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int i = tid + 256 * q, r = i >> 2, c4 = i & 3;
      sta[q] = *reinterpret_cast<const f32x4*>(a0 + r * Np + k0 + 4 * c4);
      stb[q] = *reinterpret_cast<const f32x4*>(b0 + r * Np + k0 + 4 * c4);
    }
  };
  auto put = [&](int buf) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int i = tid + 256 * q, r = i >> 2, c4 = i & 3;
      *reinterpret_cast<f32x4*>(&sA[buf][r * FC_P + 4 * c4]) = sta[q];
      *reinterpret_cast<f32x4*>(&sB[buf][r * FC_P + 4 * c4]) = stb[q];
    }
  };
  f32x16 acc[2][2] = {{f32x16{}, f32x16{}}, {f32x16{}, f32x16{}}};
  const int nk = (int)(Np / FC_K);
  fetch(0);
  put(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) fetch((int64_t)(kt + 1) * FC_K);
    f32x4 fa[2][2], fb[2][2];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        fa[s][h] = *reinterpret_cast<const f32x4*>(&sA[buf][(wr + 32 * s + n) * FC_P + 8 * g + 4 * h]);
        fb[s][h] = *reinterpret_cast<const f32x4*>(&sB[buf][(wc + 32 * s + n) * FC_P + 8 * g + 4 * h]);
      }
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int si = 0; si < 2; ++si)
#pragma unroll
          for (int sj = 0; sj < 2; ++sj) acc[si][sj] = mfma32f(fa[si][h][e], fb[sj][h][e], acc[si][sj]);
    if (kt + 1 < nk) {                               // buffer buf ^ 1 held slab kt - 1, read by every wave before the last barrier
      put(buf ^ 1);
      __syncthreads();
    }
  }
  const int64_t i0 = (int64_t)blockIdx.y * FC_T + wr, j0 = (int64_t)blockIdx.x * FC_T + wc;
#pragma unroll
  for (int si = 0; si < 2; ++si)
#pragma unroll
    for (int sj = 0; sj < 2; ++sj) {
      const int64_t j = j0 + 32 * sj + n;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t i = i0 + 32 * si + 8 * (v >> 2) + 4 * g + (v & 3);
        if (i < N && j < N) X[bc * plane + i * Np + j] = acc[si][sj][v];
      }
    }
}

// K3: tile = output row i, columns j0 .. j0 + 31: LayerNorm of X's 128 channels and of z's, then out = sigmoid(W_og
// LN(z)) * (W_o LN(X)) [+ z], the two GEMMs' chains interleaved.
__global__ void __launch_bounds__(64 * FM_NW) trimul_k3_f32m(const float* zin, float* out, const float* __restrict__ X,
                                                             const float* __restrict__ ln_in_w, const float* __restrict__ ln_in_b,
                                                             const float* __restrict__ ln_out_w, const float* __restrict__ ln_out_b, float eps,
                                                             const float* __restrict__ w_o, const float* __restrict__ w_og, int64_t N, int64_t Np,
                                                             int residual) {
  __shared__ __attribute__((aligned(16))) float sW[2][2][32 * RTF_WP];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, n = l & 31, g = l >> 5;
  const int64_t b = blockIdx.y, tpr = cdiv(N, 32), tile = (int64_t)blockIdx.x * FM_NW + wave;
  const int64_t i = tile / tpr, j = (tile % tpr) * 32 + n;
  const bool live = i < N && j < N;
  const int64_t pix = (b * N + i) * N + j, plane = Np * Np;
  f32x4 st[2][1024 / (64 * FM_NW)];
  rtf_fetch<64 * FM_NW>(w_o, 0, tid, st[0]);
  rtf_fetch<64 * FM_NW>(w_og, 0, tid, st[1]);
  float xo[64], zn[64];
  {
    const float* xp = X + (b * RT_C + 64 * g) * plane + (live ? i * Np + j : 0);
#pragma unroll
    for (int k = 0; k < 64; ++k) xo[k] = live ? xp[k * plane] : 0.0f;
  }
  rtf_norm(g, ln_out_w, ln_out_b, eps, xo);
  rtf_ln(zin + (live ? pix : 0) * RT_C, live, g, ln_in_w, ln_in_b, eps, zn);
  rtf_put<64 * FM_NW>(sW[0][0], tid, st[0]);
  rtf_put<64 * FM_NW>(sW[0][1], tid, st[1]);
  __syncthreads();
  for (int cb = 0; cb < 4; ++cb) {
    const int buf = cb & 1;
    if (cb + 1 < 4) {
      rtf_fetch<64 * FM_NW>(w_o, 32 * (cb + 1), tid, st[0]);
      rtf_fetch<64 * FM_NW>(w_og, 32 * (cb + 1), tid, st[1]);
    }
    const float* wo_r = &sW[buf][0][n * RTF_WP + 64 * g];
    const float* wg_r = &sW[buf][1][n * RTF_WP + 64 * g];
    f32x16 o = f32x16{}, gt = f32x16{};
#pragma unroll
    for (int s4 = 0; s4 < 16; ++s4) {
      const f32x4 fo = *reinterpret_cast<const f32x4*>(wo_r + 4 * s4);
      const f32x4 fg = *reinterpret_cast<const f32x4*>(wg_r + 4 * s4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o = mfma32f(fo[e], xo[4 * s4 + e], o);
        gt = mfma32f(fg[e], zn[4 * s4 + e], gt);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (live) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t oo = pix * RT_C + 32 * cb + 8 * q + 4 * g;     // channels of registers 4 q .. 4 q + 3
        f32x4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = sigmoid_exact(gt[4 * q + e]) * o[4 * q + e];
        if (residual) {
          const f32x4 r = *reinterpret_cast<const f32x4*>(zin + oo);
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] += r[e];
        }
        *reinterpret_cast<f32x4*>(out + oo) = y;
      }
    }
    if (cb + 1 < 4) {
      rtf_put<64 * FM_NW>(sW[buf ^ 1][0], tid, st[0]);
      rtf_put<64 * FM_NW>(sW[buf ^ 1][1], tid, st[1]);
      __syncthreads();
    }
  }
}

static int64_t padded(int64_t n) { return cdiv(n, TM_TILE) * TM_TILE; }
// The contraction's depth: the pair axis rounded up to 64 (two 32-deep slabs per step of its loop); the planes are zero from N
// to Np along it, so the slabs past the depth would add only zero products.
static int64_t depth(int64_t n) { return cdiv(n, 64) * 64; }

// The contraction of operand planes holding cpl channels (A rows a0 .. a0 + Ra - 1 of a plane of La rows, B whole) into X
// (Ra rows, all 128 channels; these planes' channel c at cx0 + c): persistent, a multiple of 8 workgroups.
static int contract_launch(hipStream_t st, const uint16_t* pa, const uint16_t* pb, uint16_t* X, int64_t Np, int64_t Nk, int64_t B, int cpl, int64_t La,
                           int64_t a0, int64_t Ra, int cx0, char* err, size_t errlen) {
  if (cpl != 32 && cpl != 64 && cpl != TM_C) return fail(err, errlen, FPF_E_ARGS, "operand planes of %d channels (32, 64 or 128)", cpl);
  const int64_t tiles = cdiv(Ra, CB_T) * cdiv(Np, CB_T) * B * cpl;
  const int64_t grid = std::min<int64_t>(cdiv(tiles, 8), std::max(num_cus() / 8, 1)) * 8;
  if (Nk <= 0 || Nk % 64 || Nk > Np) return fail(err, errlen, FPF_E_ARGS, "contraction depth %lld of a %lld plane", (long long)Nk, (long long)Np);
  if ((cdiv(cdiv(tiles, 8), grid / 8) + 1) * (Nk / CB_K) >= (int64_t(1) << 31)) return fail(err, errlen, FPF_E_SHAPE, "contraction slab count above 2^31");
  auto kern = cpl == 32 ? trimul_contract_bf16_256<32> : cpl == 64 ? trimul_contract_bf16_256<64> : trimul_contract_bf16_256<TM_C>;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(256), 0, st, pa, pb, X, Np, Nk, B * cpl, La, a0, Ra, cx0);
  return launched(err, errlen, "trimul_contract_bf16_256");
}
// The contraction tile: 256 at every n (a padded extent of an odd multiple of 128 ends with half-inside tiles).
static int64_t ctile(int64_t n) { (void)n; return CB_T; }

// Contraction -> K3 of the bf16 path for output rows [row0, row0 + rows), from whole A and B planes: A rows a0 .. a0 + Ra - 1
// (the tile-aligned cover of the row block) into an X plane of Ra rows.  The whole op is row0 = 0, rows = N, Ra = Np.
static int k3_launch(const FpfTrimulArgs* a, hipStream_t st, const uint16_t* X, int64_t row0, int64_t rows, int64_t a0, int64_t Ra, char* err,
                     size_t errlen);

static int bf16_rows(const FpfTrimulArgs* a, hipStream_t st, const uint16_t* pa, const uint16_t* pb, uint16_t* X, int64_t row0, int64_t rows,
                     char* err, size_t errlen) {
  const int64_t N = a->n, Np = padded(N), B = a->batch, T = ctile(N);
  // the row block's cover by contraction tiles, capped at the plane (Np, a multiple of 128, may end half way into a tile)
  const int64_t a0 = row0 / T * T, Ra = std::min<int64_t>(cdiv(row0 + rows, T) * T, Np) - a0;
  const int64_t k3_tiles = B * rows * cdiv(N, 32);
  if (!rt_tiles_ok(k3_tiles)) return fail(err, errlen, FPF_E_SHAPE, "2^31 or more 32-pixel tiles");
  int rc = contract_launch(st, pa, pb, X, Np, depth(N), B, TM_C, Np, a0, Ra, 0, err, errlen);
  if (rc) return rc;
  return k3_launch(a, st, X, row0, rows, a0, Ra, err, errlen);
}

// K3 (LN_out(X) + W_o x sigmoid(gate) + residual) on output rows row0 .. row0 + rows - 1, from X's rows a0 .. a0 + Ra - 1
static int k3_launch(const FpfTrimulArgs* a, hipStream_t st, const uint16_t* X, int64_t row0, int64_t rows, int64_t a0, int64_t Ra, char* err,
                     size_t errlen) {
  const int64_t N = a->n, Np = padded(N), B = a->batch;
  const int64_t k3_tiles = B * rows * cdiv(N, 32);
  const unsigned k3_grid = (unsigned)std::min<int64_t>(num_cus(), cdiv(k3_tiles, RT_WAVES));
  hipLaunchKernelGGL(a->dtype == FPF_DT_F32Z_BF16 ? trimul_k3_bf16<true> : trimul_k3_bf16<false>, dim3(k3_grid), dim3(512), 0, st, a->z, a->out, X,
                     a->ln_in_w, a->ln_in_b, a->ln_out_w, a->ln_out_b, a->eps, (const uint16_t*)a->w_o, (const uint16_t*)a->w_og, N, Np, B,
                     a->residual, row0, rows, a0, Ra);
  return launched(err, errlen, "trimul_k3_bf16");
}

// K1: both planes (LN_in + four gated projections + mask), into pa / pb: channel blocks cb0 .. cb0 + ncb - 1 (32 channels
// each) as planes of 32 ncb channels; the whole op: all four into planes of 128.
static int bf16_planes(const FpfTrimulArgs* a, hipStream_t st, uint16_t* pa, uint16_t* pb, char* err, size_t errlen, int cb0 = 0, int ncb = 4) {
  const int64_t N = a->n, Np = padded(N), B = a->batch;
  const int64_t k1_tiles = B * Np * (Np / 32);
  if (!rt_tiles_ok(k1_tiles)) return fail(err, errlen, FPF_E_SHAPE, "2^31 or more 32-pixel tiles");
  if (ncb != 1 && ncb != 2 && ncb != 4) return fail(err, errlen, FPF_E_ARGS, "K1 writes 1, 2 or 4 channel blocks (got %d)", ncb);
  const unsigned k1_grid = (unsigned)std::min<int64_t>(num_cus(), cdiv(k1_tiles, RT_WAVES));
  const bool f = a->dtype == FPF_DT_F32Z_BF16;
  const double plane_bytes = 2.0 * (double)B * (32 * ncb) * (double)Np * (double)Np * 2;      // A and B planes, bf16
  const bool nt = plane_bytes > 256.0 * 1024 * 1024;                                           // above the last-level cache
#define FPF_K1(Z, C) (nt ? trimul_k1_bf16<Z, C, true> : trimul_k1_bf16<Z, C, false>)
  auto kern = ncb == 4 ? (f ? FPF_K1(true, 4) : FPF_K1(false, 4))
                       : ncb == 2 ? (f ? FPF_K1(true, 2) : FPF_K1(false, 2)) : (f ? FPF_K1(true, 1) : FPF_K1(false, 1));
#undef FPF_K1
  hipLaunchKernelGGL(kern, dim3(k1_grid), dim3(512), 0, st, a->z, a->mask, a->ln_in_w, a->ln_in_b, a->eps, (const uint16_t*)a->w_ap,
                     (const uint16_t*)a->w_ag, (const uint16_t*)a->w_bp, (const uint16_t*)a->w_bg, pa, pb, N, Np, B, a->outgoing, cb0);
  return launched(err, errlen, "trimul_k1_bf16");
}

static int bf16_checks(const FpfTrimulArgs* a, char* err, size_t errlen) {
  if (a->c_z != TM_C || a->c_h != TM_C) return fail(err, errlen, FPF_E_SHAPE, "bf16 trimul serves c_z = c_h = 128 (got %d, %d)", a->c_z, a->c_h);
  if (!aligned16(a->z) || !aligned16(a->out) || !aligned16(a->w_ag) || !aligned16(a->w_ap) || !aligned16(a->w_bg) || !aligned16(a->w_bp) ||
      !aligned16(a->w_o) || !aligned16(a->w_og))
    return fail(err, errlen, FPF_E_ALIGN, "operands must be 16-byte aligned");
  return FPF_OK;
}

}  // namespace fpf

extern "C" size_t fpf_trimul_fixed_bytes(int64_t batch, int64_t n, int32_t c_h, int32_t dtype) {
  const int64_t Np = fpf::padded(n);
  return dtype == FPF_DT_BF16 ? (size_t)2 * (size_t)batch * (size_t)c_h * (size_t)Np * (size_t)Np * 2 : 0;
}

extern "C" size_t fpf_trimul_rows_workspace_bytes(int64_t batch, int64_t n, int64_t rows, int32_t c_h, int32_t dtype) {
  if (dtype != FPF_DT_BF16 || rows <= 0 || n <= 0) return 0;
  // the X plane of a row block's tile-aligned cover: at most rows rounded up to the tile, plus one tile, capped at the plane
  const int64_t Np = fpf::padded(n), T = fpf::ctile(n), Ra = std::min<int64_t>(fpf::cdiv(std::min(rows, n), T) * T + T, Np);
  return (size_t)batch * (size_t)c_h * (size_t)Ra * (size_t)Np * 2;
}

extern "C" int fpf_trimul_fixed_fwd(const FpfTrimulArgs* a, void* fixed_out, void* stream, char* err, size_t errlen) {
  using namespace fpf;
  FPF_CHECK_VERSION(a);
  if (!a->z || !a->ln_in_w || !a->ln_in_b || !a->w_ag || !a->w_ap || !a->w_bg || !a->w_bp || !fixed_out)
    return fail(err, errlen, FPF_E_ARGS, "z / ln_in / the four projection weights / fixed_out is NULL");
  if (a->dtype != FPF_DT_BF16) return fail(err, errlen, FPF_E_DTYPE, "the rows mode serves the bf16 trimul");
  if (a->batch <= 0 || a->n <= 0) return a->batch == 0 || a->n == 0 ? FPF_OK : fail(err, errlen, FPF_E_SHAPE, "batch / n negative");
  if (a->batch > 65535) return fail(err, errlen, FPF_E_SHAPE, "batch above 65535");
  if (a->c_z != TM_C || a->c_h != TM_C) return fail(err, errlen, FPF_E_SHAPE, "bf16 trimul serves c_z = c_h = 128 (got %d, %d)", a->c_z, a->c_h);
  if (!aligned16(a->z) || !aligned16(fixed_out) || !aligned16(a->w_ag) || !aligned16(a->w_ap) || !aligned16(a->w_bg) || !aligned16(a->w_bp))
    return fail(err, errlen, FPF_E_ALIGN, "operands must be 16-byte aligned");
  const int64_t Np = padded(a->n);
  uint16_t* pa = static_cast<uint16_t*>(fixed_out);
  return bf16_planes(a, static_cast<hipStream_t>(stream), pa, pa + a->batch * TM_C * Np * Np, err, errlen);
}

extern "C" size_t fpf_trimul_workspace_bytes(int64_t batch, int64_t n, int32_t c_z, int32_t c_h, int32_t dtype) {
  (void)c_z;
  const int64_t Np = fpf::padded(n);
  const size_t elt = dtype == FPF_DT_F32 ? 4 : 2;
  return (size_t)3 * (size_t)batch * (size_t)c_h * (size_t)Np * (size_t)Np * elt;
}

extern "C" int fpf_trimul_fwd(const FpfTrimulArgs* a, void* stream, char* err, size_t errlen) {
  using namespace fpf;
  FPF_CHECK_VERSION(a);
  if (!a->z || !a->out || !a->ln_in_w || !a->ln_in_b || !a->ln_out_w || !a->ln_out_b || !a->w_ag || !a->w_ap || !a->w_bg || !a->w_bp ||
      !a->w_o || !a->w_og)
    return fail(err, errlen, FPF_E_ARGS, "a required pointer is NULL (z, out, the ten weights)");
  if (a->batch <= 0 || a->n <= 0) return a->batch == 0 || a->n == 0 ? FPF_OK : fail(err, errlen, FPF_E_SHAPE, "batch / n negative");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t N = a->n, Np = padded(N), B = a->batch;
  if (B > 65535) return fail(err, errlen, FPF_E_SHAPE, "batch above 65535");
  if (a->rows != 0 || a->row0 != 0 || a->fixed_in) {    // rows mode: output rows [row0, row0 + rows) from the planes in fixed_in
    if (a->dtype != FPF_DT_BF16) return fail(err, errlen, FPF_E_DTYPE, "the rows mode serves the bf16 trimul");
    if (a->rows <= 0 || a->row0 < 0 || a->row0 + a->rows > N)
      return fail(err, errlen, FPF_E_SHAPE, "rows [%lld, %lld) outside [0, %lld)", (long long)a->row0, (long long)(a->row0 + a->rows), (long long)N);
    if (!a->fixed_in) return fail(err, errlen, FPF_E_ARGS, "the rows mode takes the A | B planes in fixed_in (fpf_trimul_fixed_fwd)");
    int rc = bf16_checks(a, err, errlen);
    if (rc) return rc;
    const size_t need = fpf_trimul_rows_workspace_bytes(B, N, a->rows, a->c_h, a->dtype);
    if (!a->workspace || a->workspace_bytes < need)
      return fail(err, errlen, FPF_E_WORKSPACE, "workspace %zu < %zu bytes", (size_t)a->workspace_bytes, need);
    if (!aligned16(a->workspace) || !aligned16(a->fixed_in)) return fail(err, errlen, FPF_E_ALIGN, "workspace / fixed_in must be 16-byte aligned");
    const uint16_t* pa = static_cast<const uint16_t*>(a->fixed_in);
    return bf16_rows(a, st, pa, pa + B * TM_C * Np * Np, static_cast<uint16_t*>(a->workspace), a->row0, a->rows, err, errlen);
  }
  const size_t need = fpf_trimul_workspace_bytes(a->batch, a->n, a->c_z, a->c_h, a->dtype);
  if (!a->workspace || a->workspace_bytes < need)
    return fail(err, errlen, FPF_E_WORKSPACE, "workspace %zu < %zu bytes", (size_t)a->workspace_bytes, need);
  if (a->dtype == FPF_DT_BF16 || a->dtype == FPF_DT_F32Z_BF16) {    // bf16 planes; z / out bf16, or fp32 (the fp32-resident form)
    int rc = bf16_checks(a, err, errlen);
    if (rc) return rc;
    if (!aligned16(a->workspace)) return fail(err, errlen, FPF_E_ALIGN, "operands must be 16-byte aligned");
    uint16_t* pa = static_cast<uint16_t*>(a->workspace);
    uint16_t* pb = pa + B * TM_C * Np * Np;
    uint16_t* X = pb + B * TM_C * Np * Np;
    rc = bf16_planes(a, st, pa, pb, err, errlen);
    if (rc) return rc;
    return bf16_rows(a, st, pa, pb, X, 0, N, err, errlen);
  }
  if (a->dtype == FPF_DT_F32) {
    if (a->c_z > F_CM || a->c_h > F_CM) return fail(err, errlen, FPF_E_SHAPE, "fp32 trimul serves c_z, c_h <= %d", F_CM);
    float* pa = static_cast<float*>(a->workspace);
    float* pb = pa + B * a->c_h * Np * Np;
    float* X = pb + B * a->c_h * Np * Np;
    if (a->c_z == TM_C && a->c_h == TM_C && aligned16(a->z) && aligned16(a->out) && aligned16(a->workspace) && aligned16(a->w_ap) &&
        aligned16(a->w_ag) && aligned16(a->w_bp) && aligned16(a->w_bg) && aligned16(a->w_o) && aligned16(a->w_og) &&
        (!a->ln_in_w || aligned16(a->ln_in_w)) && (!a->ln_in_b || aligned16(a->ln_in_b)) && (!a->ln_out_w || aligned16(a->ln_out_w)) &&
        (!a->ln_out_b || aligned16(a->ln_out_b))) {   // the matrix-core kernels
      hipLaunchKernelGGL(trimul_k1_f32m, dim3((unsigned)(Np * (Np / 32) / FM_NW), (unsigned)B), dim3(64 * FM_NW), 0, st, (const float*)a->z,
                         a->mask, a->ln_in_w, a->ln_in_b, a->eps, (const float*)a->w_ap, (const float*)a->w_ag, (const float*)a->w_bp,
                         (const float*)a->w_bg, pa, pb, N, Np, a->outgoing);
      int rc = launched(err, errlen, "trimul_k1_f32m");
      if (rc) return rc;
      hipLaunchKernelGGL(trimul_contract_f32m, dim3((unsigned)(Np / FC_T), (unsigned)(Np / FC_T), (unsigned)(B * TM_C)), dim3(256), 0, st, pa,
                         pb, X, Np, N);
      rc = launched(err, errlen, "trimul_contract_f32m");
      if (rc) return rc;
      hipLaunchKernelGGL(trimul_k3_f32m, dim3((unsigned)cdiv(N * cdiv(N, 32), FM_NW), (unsigned)B), dim3(64 * FM_NW), 0, st, (const float*)a->z,
                         (float*)a->out, X, a->ln_in_w, a->ln_in_b, a->ln_out_w, a->ln_out_b, a->eps, (const float*)a->w_o,
                         (const float*)a->w_og, N, Np, a->residual);
      return launched(err, errlen, "trimul_k3_f32m");
    }
    hipLaunchKernelGGL(trimul_k1_f32, dim3((unsigned)(Np * Np / F_R), (unsigned)B), dim3(256), 0, st, (const float*)a->z, a->mask, a->ln_in_w,
                       a->ln_in_b, a->eps, (const float*)a->w_ap, (const float*)a->w_ag, (const float*)a->w_bp, (const float*)a->w_bg, pa, pb, N,
                       Np, a->c_z, a->c_h, a->outgoing);
    int rc = launched(err, errlen, "trimul_k1_f32");
    if (rc) return rc;
    hipLaunchKernelGGL(trimul_contract_f32, dim3((unsigned)(Np / SG_T), (unsigned)(Np / SG_T), (unsigned)(B * a->c_h)), dim3(256), 0, st, pa,
                       pb, X, Np, N);
    rc = launched(err, errlen, "trimul_contract_f32");
    if (rc) return rc;
    hipLaunchKernelGGL(trimul_k3_f32, dim3((unsigned)(Np * Np / F_R), (unsigned)B), dim3(256), 0, st, (const float*)a->z, (float*)a->out, X,
                       a->ln_in_w, a->ln_in_b, a->ln_out_w, a->ln_out_b, a->eps, (const float*)a->w_o, (const float*)a->w_og, N, Np, a->c_z,
                       a->c_h, a->residual);
    return launched(err, errlen, "trimul_k3_f32");
  }
  return fail(err, errlen, FPF_E_DTYPE, "dtype %d", a->dtype);
}

// ---------------------------------------------------------------------------------------------------------------- channels mode
// The product plane X is built channel block by channel block (common/opt_core/opt_core/mem/chunk.py:542-552, mode
// "channels"): per block of `chunk` hidden channels, K1 writes the A / B planes of those channels only (LN_in recomputed,
// the block's projection columns), and the contraction writes those channels of the one full X; K3 then runs over all rows.
// Each channel of X is computed by the same instructions on the same values as in the whole op (K1's 32-channel blocks
// and the contraction's per-channel products are independent of one another), so the result equals fpf_trimul_fwd bitwise.
// Held: X (all channels) + two planes of `chunk` channels, against the whole op's three 128-channel planes.
namespace fpf {
static int64_t channel_block(int64_t chunk) { return chunk >= TM_C ? TM_C : chunk >= 64 ? 64 : 32; }
}  // namespace fpf

extern "C" size_t fpf_trimul_channels_workspace_bytes(int64_t batch, int64_t n, int64_t chunk, int32_t c_h, int32_t dtype) {
  if ((dtype != FPF_DT_BF16 && dtype != FPF_DT_F32Z_BF16) || c_h != fpf::TM_C || chunk <= 0 || n <= 0 || batch <= 0) return 0;
  const int64_t Np = fpf::padded(n), cpl = fpf::channel_block(chunk);
  return (size_t)batch * (size_t)(fpf::TM_C + 2 * cpl) * (size_t)Np * (size_t)Np * 2;
}

extern "C" int fpf_trimul_channels_fwd(const FpfTrimulArgs* a, int64_t chunk, void* stream, char* err, size_t errlen) {
  using namespace fpf;
  FPF_CHECK_VERSION(a);
  if (!a->z || !a->out || !a->ln_in_w || !a->ln_in_b || !a->ln_out_w || !a->ln_out_b || !a->w_ag || !a->w_ap || !a->w_bg || !a->w_bp ||
      !a->w_o || !a->w_og)
    return fail(err, errlen, FPF_E_ARGS, "a required pointer is NULL (z, out, the ten weights)");
  if (a->rows || a->row0 || a->fixed_in) return fail(err, errlen, FPF_E_ARGS, "the channels mode runs every row (rows mode: fpf_trimul_fwd)");
  if (a->dtype != FPF_DT_BF16 && a->dtype != FPF_DT_F32Z_BF16) return fail(err, errlen, FPF_E_DTYPE, "the channels mode serves the bf16 trimul");
  if (chunk <= 0) return fail(err, errlen, FPF_E_ARGS, "chunk %lld: a positive channel count", (long long)chunk);
  if (a->batch <= 0 || a->n <= 0) return a->batch == 0 || a->n == 0 ? FPF_OK : fail(err, errlen, FPF_E_SHAPE, "batch / n negative");
  if (a->batch > 65535) return fail(err, errlen, FPF_E_SHAPE, "batch above 65535");
  int rc = bf16_checks(a, err, errlen);
  if (rc) return rc;
  const size_t need = fpf_trimul_channels_workspace_bytes(a->batch, a->n, chunk, a->c_h, a->dtype);
  if (!a->workspace || a->workspace_bytes < need)
    return fail(err, errlen, FPF_E_WORKSPACE, "workspace %zu < %zu bytes", (size_t)a->workspace_bytes, need);
  if (!aligned16(a->workspace)) return fail(err, errlen, FPF_E_ALIGN, "operands must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t N = a->n, Np = padded(N), B = a->batch, cpl = channel_block(chunk);
  uint16_t* X = static_cast<uint16_t*>(a->workspace);
  uint16_t* pa = X + B * TM_C * Np * Np;
  uint16_t* pb = pa + B * cpl * Np * Np;
  for (int64_t c0 = 0; c0 < TM_C; c0 += cpl) {
    rc = bf16_planes(a, st, pa, pb, err, errlen, (int)(c0 / 32), (int)(cpl / 32));
    if (rc) return rc;
    rc = contract_launch(st, pa, pb, X, Np, depth(N), B, (int)cpl, Np, 0, Np, (int)c0, err, errlen);
    if (rc) return rc;
  }
  return k3_launch(a, st, X, 0, N, 0, Np, err, errlen);
}

// ---------------------------------------------------------------------------------------------------------------- no-allocation entry
// fpf_trimul_fwd for callers that cannot allocate (graph capture, serving loops, harnesses that forbid hipMalloc): the
// workspace is a file-scope device array, `scratch`, which every GPU the library runs on holds until the process ends.  In
// host code `scratch` names a host-side stand-in, not device memory: its device address is taken once per device with that
// device current (hipGetSymbolAddress) and only that address is handed to kernels.  The K1 planes need no clearing (K1
// writes every padded element, zeros outside the N x N pixels), so nothing is reset between calls.  Calls that overlap on
// one GPU (two streams, two host threads) share the array and race.
namespace fpf {
static __device__ __align__(256) unsigned char scratch[FPF_TRIMUL_NOALLOC_SCRATCH_BYTES];
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64];

// The device address of this device's `scratch` (looked up on its first use here, with the device current).
static int scratch_address(void** out, char* err, size_t errlen) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(err, errlen, FPF_E_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= 64) return fail(err, errlen, FPF_E_ARGS, "device %d outside the 64 this library tracks", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return fail(err, errlen, FPF_E_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return FPF_OK;
}
}  // namespace fpf

extern "C" int fpf_trimul_fwd_noalloc(const FpfTrimulArgs* a, void* stream, char* err, size_t errlen) {
  using namespace fpf;
  FPF_CHECK_VERSION(a);
  if (a->workspace || a->workspace_bytes)
    return fail(err, errlen, FPF_E_ARGS, "the no-allocation entry uses the library's static scratch: pass workspace NULL, workspace_bytes 0");
  if (a->rows || a->row0 || a->fixed_in) return fail(err, errlen, FPF_E_ARGS, "the no-allocation entry runs the whole op (rows mode: fpf_trimul_fwd)");
  if (a->batch < 0 || a->n < 0) return fail(err, errlen, FPF_E_SHAPE, "batch / n negative");
  const size_t need = fpf_trimul_workspace_bytes(a->batch, a->n, a->c_z, a->c_h, a->dtype);
  if (need > (size_t)FPF_TRIMUL_NOALLOC_SCRATCH_BYTES)
    return fail(err, errlen, FPF_E_WORKSPACE, "needs %zu workspace bytes, above the %zu-byte static scratch (bf16, B = 1: N <= 256)", need,
                (size_t)FPF_TRIMUL_NOALLOC_SCRATCH_BYTES);
  // the scratch address is the current device's: a stream of another device would run the kernels there with this device's
  // address, so such a stream is refused before anything is launched (the null stream is the current device's)
  if (stream) {
    int cur = 0;
    hipDevice_t sdev = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e == hipSuccess) e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev);
    if (e != hipSuccess) return fail(err, errlen, FPF_E_ARGS, "the stream's device could not be read: %s", hipGetErrorString(e));
    if ((int)sdev != cur)
      return fail(err, errlen, FPF_E_ARGS, "the stream belongs to device %d but device %d is current: make the stream's device current", (int)sdev, cur);
  }
  FpfTrimulArgs b = *a;
  const int rc = scratch_address(&b.workspace, err, errlen);
  if (rc) return rc;
  b.workspace_bytes = (size_t)FPF_TRIMUL_NOALLOC_SCRATCH_BYTES;
  return fpf_trimul_fwd(&b, stream, err, errlen);
}
