// Triangle attention: the fused block's core on the block's own operand layout (v_layout 2; V as key rows: v_layout 3), and the
// keep-bit table it reads.
// Replaces the core stage of common/opt_core/opt_core/attn/pair_fused.py:1391 (core_attention) inside tri_attn_block (:1500):
// o = softmax_j(q.k + bias, -inf at masked keys) v per (b, attention row i, head h), kernels/triattn/__init__.py:3-8; a row with
// no kept key is the uniform mean of v.
//
// Operands (written by the block's prologue): q [B, N, H, S, 32] already times scale * log2(e), k [B, N, H, S, 32], V^T
// [B, N, H, 32, S] with the keys of every 16-key block stored 0-3, 8-11, 4-7, 12-15 (the order in which the S^T MFMA's output
// registers hold P), fp32 bias planes [B, H] of S x S times log2(e) in 32 x 32 register-order blocks (bias_blk_off):
// logits are in log2 units throughout.
//
// Work split: a work item = TA_R pair rows x 32 NW queries x one (b, h); a wave = 32 queries of the TA_R rows (lane n = query,
// lane group g = key half).  The TA_R rows share the bias (it does not depend on i): each wave loads its 32 x 32 fp32 bias
// sub-tile once into registers (four contiguous 1 KB reads) and starts all TA_R rows' S^T = K Q^T accumulators
// (v_mfma_f32_32x32x16_bf16) from it.  K and V^T tiles of 64 keys go global -> LDS by DMA (global_load_lds_dwordx4) through
// a ring of TA_NB buffers, in XOR-swizzled 16-byte chunks (K: chunk c of key k at c ^ ((k >> 2) & 3); V^T: chunk c of row d
// at c ^ ((d >> 1) & 7)), so every fragment read is a conflict-free 16-byte read; all TA_R rows' tiles are shared by the NW
// waves.  Workgroups are persistent and walk strided sequences of items (the next item's first tiles, bias and q are
// fetched during the current item's last tiles).
//
// The step pipeline.  The key loop is a sequence of steps (t, r) over 32-key sub-tiles t and rows r.  Step (t, r) turns
// the row's S^T sub-tile (already in registers) into P = exp2(s) rounded to bf16 and adds those bf16 values to the row's
// running sums (softmax_step).  In the same basic block it issues the MFMAs of the PREVIOUS step -- that row's O^T +=
// V^T P^T with the P computed one step earlier, and the same row's S^T of the next sub-tile -- so the matrix core works
// while the wave computes exponentials (a wave issues in order: an MFMA right behind the exponentials it consumes would
// stall it).  The MFMAs and the softmax arithmetic are interleaved by sched_group_barrier.
//
// The softmax reference (the max subtracted before exp2) is 0: exact whenever a query's row sum lies in [2^-32, 2^64),
// which one test per query at the end of the item checks.  A work item with a query outside that range is recomputed by
// the fallback kernel, which repeats the sums in a first pass and uses the query's max as the reference where they are
// out of range (and 0 elsewhere, so both kernels produce the same bits for every other query).  Tiles where every key of
// the TA_R rows is kept and no row is dead run with no mask code at all; the keep bits come from a table built once per
// call (triattn_keep_bits_u8 / triattn_keep_bits), so the key loop never reads the mask.
#include <algorithm>

#include "triattn.h"

namespace fpf {

// ---------------------------------------------------------------------------------------------------------------- keep table
// One wave per (b, attention row i): 64 keys per ballot, 16 mask loads in flight.  The table layout is in triattn.h.
__global__ void __launch_bounds__(256) triattn_keep_bits(const void* __restrict__ mask, int mask_f32, int64_t ms0, int64_t ms1, int64_t ms2,
                                                           int64_t B, int64_t N, int64_t S, int64_t Sv, uint64_t* __restrict__ keep) {
  const int l = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= B * N) return;
  const int64_t b = row / N, i = row - b * N;
  const int nw = (int)(S >> 6);
  uint64_t* out = keep + row * keep_words(S);
  const int64_t base = b * ms0 + i * ms1;
  uint64_t any = 0, all = ~0ull, mine0 = 0, mine1 = 0, real0 = 0, real1 = 0;   // words l and 64 + l of the row (and of real keys)
  for (int c0 = 0; c0 < nw; c0 += 16) {
    bool k[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int64_t key = (int64_t)64 * (c0 + u) + l;
      const int64_t off = base + (key < Sv ? key : 0) * ms2;
      k[u] = key < Sv && (!mask || (mask_f32 ? static_cast<const float*>(mask)[off] != 0.f : static_cast<const uint8_t*>(mask)[off] != 0));
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int c = c0 + u;
      if (c >= nw) break;
      const uint64_t bal = __ballot(k[u]);
      const uint64_t real = __ballot((int64_t)64 * c + l < Sv);
      any |= bal;
      all &= bal;
      if ((c & 63) == l) {
        if (c < 64) mine0 = bal, real0 = real;
        else mine1 = bal, real1 = real;
      }
    }
  }
  if (l < nw) out[1 + l] = any ? mine0 : real0;
  if (64 + l < nw) out[65 + l] = any ? mine1 : real1;
  if (l == 0) out[0] = (any ? TK_ALIVE : 0) | (all == ~0ull ? TK_FULL : 0);
}

// The same table from a u8 mask with contiguous keys and 16-byte aligned rows: lane l loads keys 1024 c + 16 l .. +15 in one
// 16-byte load, turns each byte into its keep bit with word arithmetic, and lanes 4 T .. 4 T + 3 assemble word T.
__device__ __forceinline__ uint32_t kb_nibble(uint32_t w) {    // bit e = (byte e of w != 0), e = 0 .. 3
  const uint32_t hi = (((w & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | w) & 0x80808080u;   // bit 8 e + 7: byte e is nonzero
  return ((hi >> 7) * 0x10204080u) >> 28;                   // bits 0, 8, 16, 24 gathered to 28 .. 31 (no two products meet)
}
// Sv is a multiple of 16 here (the launcher's condition), so no 16-byte load straddles the end of the real keys.
__global__ void __launch_bounds__(256) triattn_keep_bits_u8(const uint8_t* __restrict__ mask, int64_t ms0, int64_t ms1, int64_t B, int64_t N,
                                                              int64_t S, int64_t Sv, uint64_t* __restrict__ keep) {
  const int l = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= B * N) return;
  const int64_t b = row / N, i = row - b * N;
  const uint8_t* src = mask + b * ms0 + i * ms1;
  uint64_t* out = keep + row * keep_words(S);
  bool any = false, all = Sv == S;                          // a padded row is never FULL
  for (int64_t c0 = 0; c0 < S; c0 += 1024) {
    const int64_t k0 = c0 + 16 * l;
    const bool real = k0 < Sv, inrow = k0 < S;
    const u32x4 v = real ? *reinterpret_cast<const u32x4*>(src + k0) : u32x4{0, 0, 0, 0};
    const uint32_t piece = kb_nibble(v[0]) | (kb_nibble(v[1]) << 4) | (kb_nibble(v[2]) << 8) | (kb_nibble(v[3]) << 12);
    any |= __builtin_amdgcn_ballot_w64(real && piece != 0) != 0;
    all &= __builtin_amdgcn_ballot_w64(real && piece != 0xFFFFu) == 0;
    // lanes 4 T + 1 .. 4 T + 3 hand their pieces to lane 4 T (keys 64 T + 16 .. 64 T + 63)
    const uint32_t p1 = __shfl_down(piece, 1), p2 = __shfl_down(piece, 2), p3 = __shfl_down(piece, 3);
    if ((l & 3) == 0 && inrow)
      out[1 + (c0 >> 6) + (l >> 2)] = (uint64_t)(piece | (p1 << 16)) | ((uint64_t)(p2 | (p3 << 16)) << 32);
  }
  if (!any) {                                               // no kept key: every real key's bit set (the row attends uniformly)
    for (int64_t w = l; w < S / 64; w += 64) {
      const int64_t nreal = Sv - 64 * w;
      out[1 + w] = nreal >= 64 ? ~0ull : nreal > 0 ? (1ull << nreal) - 1 : 0ull;
    }
  }
  if (l == 0) out[0] = (any ? TK_ALIVE : 0) | (all ? TK_FULL : 0);
}

// ---------------------------------------------------------------------------------------------------------------- core
constexpr int TA_OP = 40;        // LDS pitch (bf16) of the per-wave output staging rows (80 B: 16-byte aligned, few conflicts)

// One work item: TA_R pair rows x 32 NW queries x one (b, h), and the addresses its loads use.  The row-i0 bases of K, V^T
// and q and the wave's row of bias blocks are wave-uniform (scalar registers; row r adds r times the row stride, rows past N
// read row i0); q (the lane's query) and qo (its byte offset in a q row) are per lane.
struct PipeItem {
  const uint16_t* kb;
  const uint16_t* vb;
  const uint16_t* qb;
  const float* brow;               // bias block (wave's 32 queries, keys 0 .. 31); key sub-tile s adds 1024 s
  int32_t b, h, i0, nrow;          // nrow: rows of the item below N (1 .. TA_R)
  int32_t q;
  uint32_t qo;
};

// Persistent: XCD x takes the x-th eighth of the work items (one XCD works on one head and keeps its bias in L2) and its
// workgroups take every nwg-th item of that range, so the query tiles of a row group run at the same time on neighbouring
// workgroups and fetch the rows' K / V^T tiles from HBM once (a workgroup walking them back to back found them evicted by
// the other CUs' streams: 1146 against 704 MB fetched per launch at N = 768).  The K / V^T DMA ring and the bias
// double buffer run across item boundaries (the loads past an item's last tile fetch the next item's first tiles), the next
// item's q is loaded during the item's second-to-last tile, and an item's output leaves through LDS as contiguous 16-byte
// stores that drain while the next item computes.
// MASKED: the call has a keep table (without one every key is kept and the kernel carries no mask code).
template <int NW, bool MASKED, bool VROWS>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2))) triattn_core_bf16_pipe(const CoreParams p) {
  constexpr int R = TA_R;
  __shared__ __attribute__((aligned(16))) uint16_t sK[TA_NB][R][TA_KT * TA_D];
  __shared__ __attribute__((aligned(16))) uint16_t sV[TA_NB][R][TA_D * TA_KT];
  // output staging rows of the 8-wave split (the 4-wave split, two workgroups per CU, has no LDS left for them and stores
  // straight from registers)
  __shared__ __attribute__((aligned(16))) uint16_t sO[NW > 4 ? NW : 1][32 * TA_OP];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, n = l & 31, g = l >> 5;
  // the host checks that the item count fits 31 bits: the decode is 32-bit
  const uint32_t nq = (uint32_t)cdiv(p.S, 32 * NW), nr = (uint32_t)cdiv(p.N, R), H = (uint32_t)p.H;
  const uint32_t total = (uint32_t)p.B * H * nr * nq;
  const uint32_t xcd = blockIdx.x & 7, j = blockIdx.x >> 3, nwg = (gridDim.x - xcd + 7) >> 3;
  const uint32_t lo = (uint32_t)((uint64_t)xcd * total / 8), hi = (uint32_t)((uint64_t)(xcd + 1) * total / 8);
  const uint32_t w0 = lo + j;
  if (w0 >= hi) return;
  const int nT = (int)(p.S / TA_KT);
  const int32_t S = (int32_t)p.S, N = (int32_t)p.N, Sv = (int32_t)p.Sv;   // host-checked to fit 31 bits
  if (nT < 2) {                                    // a one-tile key range: every item goes to the fallback kernel
    for (uint32_t w = w0; w < hi; w += nwg)
      if (l == 0) p.redo[(size_t)w * NW + wave] = 1u;
    return;
  }

  const int wc = wave & 3;
  // koffL: the last tile's, whose key rows past Sqk re-read row Sqk - 1 (keys the keep table masks); V as key rows moves
  // like K (voffL the same for its last tile), V^T by rows of d
  uint32_t koff, koffL, voff, voffL;
  {
    const int kk = 16 * wc + (l >> 2), kc = (l & 3) ^ ((kk >> 2) & 3);
    const int kl = (int)p.Sqk - 1 - TA_KT * (nT - 1);
    koff = (uint32_t)((kk * p.ks[3] + 8 * kc) * 2);
    koffL = (uint32_t)(((kk < kl ? kk : kl) * p.ks[3] + 8 * kc) * 2);
    if constexpr (VROWS) {
      voff = (uint32_t)((kk * p.vs[3] + 8 * kc) * 2);
      voffL = (uint32_t)(((kk < kl ? kk : kl) * p.vs[3] + 8 * kc) * 2);
    } else {
      const int vd = 8 * wc + (l >> 3), vc = (l & 7) ^ ((vd >> 1) & 7);
      voff = voffL = (uint32_t)((vd * p.vs[3] + 8 * vc) * 2);
    }
  }
  // row r's byte offset from row i0, tile T's from tile 0 (32-bit: host-checked)
  const uint32_t krow = (uint32_t)(p.ks[1] * 2), vrow = (uint32_t)(p.vs[1] * 2), qrow = (uint32_t)(p.qs[1] * 2);
  const uint32_t ktile = (uint32_t)(TA_KT * p.ks[3] * 2), vtile = (uint32_t)(VROWS ? TA_KT * p.vs[3] * 2 : TA_KT * 2);
  auto row_at = [](const uint16_t* base, const PipeItem& it, int r, uint32_t stride) {
    return reinterpret_cast<const uint16_t*>(reinterpret_cast<const char*>(base) + (r < it.nrow ? r * stride : 0u));
  };
  auto item_of = [&](uint32_t w, PipeItem& it) {
    const uint32_t qt = w % nq, rg = (w / nq) % nr, bh = w / (nq * nr);
    it.b = (int32_t)(bh / H);
    it.h = (int32_t)(bh % H);
    it.i0 = (int32_t)(rg * R);
    it.nrow = N - it.i0 < R ? N - it.i0 : R;
    it.q = (int32_t)(qt * (32 * NW) + wave * 32 + n);
    uint64_t a[17] = {FPF_KARG(k),     FPF_KARG(v),     FPF_KARG(q),     FPF_KARG(bias),  FPF_KARG(ks[0]), FPF_KARG(ks[1]),
                      FPF_KARG(ks[2]), FPF_KARG(vs[0]), FPF_KARG(vs[1]), FPF_KARG(vs[2]), FPF_KARG(qs[0]), FPF_KARG(qs[1]),
                      FPF_KARG(qs[2]), FPF_KARG(qs[3]), FPF_KARG(bs[0]), FPF_KARG(bs[1]), FPF_KARG(Sqk)};
    karg_wait(a);
    const int64_t qs = it.q < (int32_t)a[16] ? it.q : 0;               // queries past q's rows read query 0 (never stored)
    const int64_t b = it.b, h = it.h, i0 = it.i0;
    it.kb = reinterpret_cast<const uint16_t*>(a[0]) + b * (int64_t)a[4] + i0 * (int64_t)a[5] + h * (int64_t)a[6];
    it.vb = reinterpret_cast<const uint16_t*>(a[1]) + b * (int64_t)a[7] + i0 * (int64_t)a[8] + h * (int64_t)a[9];
    it.qb = reinterpret_cast<const uint16_t*>(a[2]) + b * (int64_t)a[10] + i0 * (int64_t)a[11] + h * (int64_t)a[12];
    const int64_t qw = (int64_t)(it.q - n) < S ? (it.q - n) >> 5 : 0;   // the wave's query block (a wave past S reads block 0)
    it.brow = reinterpret_cast<const float*>(a[3]) + b * (int64_t)a[14] + h * (int64_t)a[15] + qw * (S >> 5) * 1024;
    it.qo = (uint32_t)((qs * (int64_t)a[13] + 8 * g) * 2);
  };
  // q of an item (the lane's query in each of the TA_R rows; rows past N read row i0, whose results are never stored):
  // 2 operations per row
  auto q_issue = [&](const PipeItem& it, u32x4 (&dst)[R][2]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint16_t* qp = row_at(it.qb, it, r, qrow);
      asm volatile("global_load_dwordx4 %0, %1, %2 offset:0" : "+v"(dst[r][0]) : "v"(it.qo), "s"(qp));
      asm volatile("global_load_dwordx4 %0, %1, %2 offset:32" : "+v"(dst[r][1]) : "v"(it.qo), "s"(qp));
    }
  };
  // DMA: chunk block c (1 KB) of each row's K tile (keys 16c .. 16c + 15) and V^T tile (rows 8c .. 8c + 7) is moved by wave
  // c (4 waves: both) or by waves c (K) and 4 + c (V^T) (8 waves).  Row bases are scalar, the in-tile byte offsets per lane fixed.
  const uint32_t kl0 = lds_addr(&sK[0][0][512 * wc]), vl0 = lds_addr(&sV[0][0][512 * wc]);
  constexpr uint32_t TILE_B = TA_KT * TA_D * 2;
  const bool v_mover = NW > 4 && wave >= 4;
  auto dma_tile = [&](const PipeItem& it, int T, int buf) {
    const uint32_t kt = (uint32_t)T * ktile, vt = (uint32_t)T * vtile;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (NW == 4 || !v_mover)
        lds_dma16_s(T == nT - 1 ? koffL : koff, row_at(it.kb, it, r, krow) + kt / 2, kl0 + (uint32_t)(buf * R + r) * TILE_B);
      if (NW == 4 || v_mover)
        lds_dma16_s(VROWS && T == nT - 1 ? voffL : voff, row_at(it.vb, it, r, vrow) + vt / 2, vl0 + (uint32_t)(buf * R + r) * TILE_B);
    }
  };
  // The wait counts below (vm_wait4<0>, vm_wait4<DMA_OPS>) assume exactly DMA_OPS operations per dma_tile and 4 per
  // bias_issue, every one issued unconditionally and in the order of the loop (the next item's q loads come after the last
  // tile's last counted wait, and the item start waits for everything): a wait counting fewer operations than were issued
  // after the load it guards would let that load land in registers already in use.
  constexpr int DMA_OPS = (NW == 4 ? 2 : 1) * R;
  // bias of the key sub-tile starting at k (keys k + 8 qd + 4 g + 0..3: D-layout rows of the S^T accumulator), four
  // contiguous 1 KB reads of its register-order block.  The previous value stays live up to here, so no S^T MFMA
  // accumulates in place over it and its registers are free for the new tuple
  const uint32_t boff = (uint32_t)l * 16;
  auto bias_issue = [&](const PipeItem& it, int64_t k, f32x4 (&dst)[4]) {
    const float* sb = it.brow + (k >> 5) * 1024;
    asm volatile("" ::"v"(dst[0]), "v"(dst[1]), "v"(dst[2]), "v"(dst[3]));
    dst[0] = gload4_async<0>(boff, sb);
    dst[1] = gload4_async<1024>(boff, sb);
    dst[2] = gload4_async<2048>(boff, sb);
    dst[3] = gload4_async<3072>(boff, sb);
  };
  // row flags / keep words of an item's TA_R rows (no mask: every key kept), read through the scalar cache: a vector load
  // here would come with a compiler-placed vmcnt wait that drains the counted transfers in flight
  const bool has_keep = MASKED && p.keep != nullptr;
  auto keep_row = [&](const PipeItem& it, int r) {
    uint64_t a[1] = {FPF_KARG(keep)};
    karg_wait(a);
    return reinterpret_cast<const uint64_t*>(a[0]) + ((int64_t)it.b * N + it.i0 + r) * keep_words(S);
  };
  auto row_flags = [&](const PipeItem& it, int r) -> uint32_t {
    if (!has_keep || r >= it.nrow) return (uint32_t)(TK_ALIVE | TK_FULL);
    return (uint32_t)sload64(keep_row(it, r));
  };
  auto keep_word = [&](const PipeItem& it, int r, int T) -> uint64_t {
    if (!has_keep || r >= it.nrow) return ~0ull;
    return sload64(keep_row(it, r) + 1 + T);
  };

  PipeItem cur, nxt;
  item_of(w0, cur);
  item_of(w0 + nwg < hi ? w0 + nwg : w0, nxt);
  f32x4 bq[2][4];                  // bias of the even / odd sub-tiles
  u32x4 qf[R][2];                  // q of the item (the next item's is loaded in the last tile, after the last read of these)
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) bq[x][qd] = f32x4{};
#pragma unroll
  for (int r = 0; r < R; ++r) qf[r][0] = qf[r][1] = u32x4{0, 0, 0, 0};
  q_issue(cur, qf);
  dma_tile(cur, 0, 0);
  bias_issue(cur, 0, bq[0]);
  bias_issue(cur, 32, bq[1]);
  dma_tile(cur, 1, 1);
  vm_wait<0>();                    // this wave's parts of tiles 0 and 1 are in; the barrier publishes every wave's
  __syncthreads();

  const int kfo0 = n * TA_D + 8 * ((g) ^ ((n >> 2) & 3));            // key n, chunk g (k-step 0); sub-tile 1 adds 32 keys
  const int kfo1 = n * TA_D + 8 * ((g + 2) ^ ((n >> 2) & 3));        // chunk g + 2 (k-step 1)
  const int vsw = (n >> 1) & 7;
  // S^T of row r = bias + K q: the first MFMA writes a new tuple (the bias tuple serves all TA_R rows; the compiler would
  // copy it into the accumulator instead), the second accumulates in place
  auto qk = [&](const u32x4& k0f, const u32x4& k1f, int r, const f32x4 (&bb)[4]) {
    f32x16 bc;
#pragma unroll
    for (int qd = 0; qd < 4; ++qd)
#pragma unroll
      for (int e = 0; e < 4; ++e) bc[4 * qd + e] = bb[qd][e];
    return mfma32(as_bf8(k1f), as_bf8(qf[r][1]), mfma32_new(as_bf8(k0f), as_bf8(qf[r][0]), bc));
  };
  // MFMA fragments of a step, read from LDS one step ahead: V^T of (row, sub-tile vsub of buffer vbuf), K of (row, sub-tile
  // ksub of buffer kbuf)
  u32x4 fv0, fv1, fk0, fk1;
  const uint32_t vo0 = VROWS ? vrows_off(l, 0) : 0u, vo2 = VROWS ? vrows_off(l, 2) : 0u;
  auto frags = [&](int vbuf, int vsub, int kbuf, int ksub, int row) {
    if constexpr (VROWS) {
      const uint16_t* vt = &sV[vbuf][row][0];
      fv0 = vrows_frag(vt, 32 * vsub, vo0, vo2);
      fv1 = vrows_frag(vt, 32 * vsub + 16, vo0, vo2);
    } else {
      const uint16_t* vt = &sV[vbuf][row][n * TA_KT];
      fv0 = *reinterpret_cast<const u32x4*>(vt + 8 * ((4 * vsub + g) ^ vsw));
      fv1 = *reinterpret_cast<const u32x4*>(vt + 8 * ((4 * vsub + 2 + g) ^ vsw));
    }
    const uint16_t* kt = &sK[kbuf][row][32 * ksub * TA_D];
    fk0 = *reinterpret_cast<const u32x4*>(kt + kfo0);
    fk1 = *reinterpret_cast<const u32x4*>(kt + kfo1);
  };

  f32x16 o[R], s[R];
  float la[R][2];                  // running row sums (reference 0) of the lane's keys
  bool dead[R];
  bool dead_any = false, all_full = true;
  uint32_t P0[8], P1[8];
  int bt = 0;                      // ring buffer of the current tile

  for (uint32_t w = w0; w < hi; w += nwg) {
    const bool has_next = w + nwg < hi;
    // ---- item start: state, flags, q, S^T of sub-tile 0 for rows 0 .. R - 2 (row R - 1's is issued by the first step).
    // The q loads (and every transfer before them) are in
    vm_wait<0>();
#pragma unroll
    for (int r = 0; r < R; ++r) asm volatile("" : "+v"(qf[r][0]), "+v"(qf[r][1]));
    {
      uint64_t m[1] = {FPF_KARG(qmul)};
      karg_wait(m);
      const float qmul = __uint_as_float((uint32_t)m[0]);
      if (qmul != 1.0f) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          qf[r][0] = scale_bf8(qf[r][0], qmul);
          qf[r][1] = scale_bf8(qf[r][1], qmul);
        }
      }
    }
    dead_any = false;
    all_full = true;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t f = row_flags(cur, r);
      dead[r] = !(f & TK_ALIVE);
      dead_any |= dead[r];
      all_full &= (f & TK_FULL) != 0;
      o[r] = f32x16{};
      la[r][0] = la[r][1] = 0.f;
    }
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) P0[jj] = 0u;     // P of "step -1" is zero: the first step's P.V MFMAs add nothing
#pragma unroll
    for (int r = 0; r < R - 1; ++r) {
      const uint16_t* kt = &sK[bt][r][0];
      s[r] = qk(*reinterpret_cast<const u32x4*>(kt + kfo0), *reinterpret_cast<const u32x4*>(kt + kfo1), r, bq[0]);
    }
    frags(bt, 1, bt, 0, R - 1);                       // step (0, 0)

    // one 64-key tile T (buffers: bt its own, bp tile T - 1's, bn tile T + 1's): six steps (sub, r); `fast`: every key of
    // the TA_R rows in this tile is kept and no row is dead (no mask code)
    auto tile = [&](bool fast, int T, int bp, int bn, const uint64_t (&kw)[R]) {
      const int64_t k0 = (int64_t)T * TA_KT;
      const bool moreT = T + 1 < nT;
      const PipeItem& nb = moreT ? cur : nxt;         // the item whose sub-tiles 2T + 2, 2T + 3 follow
      const int64_t kb2 = moreT ? k0 + TA_KT : 0;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (sub == 0 && r == 1) {
            vm_wait4<0>(bq[1][0], bq[1][1], bq[1][2], bq[1][3]);      // bias 2T + 1 (the newest load) is in
            bias_issue(nb, kb2, bq[0]);                                  // bias 2T + 2
          }
          if (sub == 1 && r == 0) {
            // every wave's part of tile T + 1 is in (each wave waited for it above), and every wave is past tile T - 1's
            // last reads (step (0, 0)): its buffer takes tile T + 2 (of this item, or of the next)
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if (T + 2 < nT) dma_tile(cur, T + 2, bp);
            else dma_tile(nxt, T + 2 - nT, bp);
          }
          if (sub == 1 && r == 1) {
            vm_wait4<DMA_OPS>(bq[0][0], bq[0][1], bq[0][2], bq[0][3]);  // bias 2T + 2 is in (tile T + 2 may be pending)
            bias_issue(nb, kb2 + 32, bq[1]);                               // bias 2T + 3
            // the next item's q: this item's last S^T (row R - 1, sub-tile 2 nT - 1) was issued by step (1, 0); the S^T
            // that steps (1, 1) and (1, 2) of the last tile compute for the next item are recomputed at its start
            if (T == nT - 1 && has_next) q_issue(nxt, qf);
          }
          // the previous step's row pr and the sub-tile nsub of the S^T its MFMAs compute (tile-relative: -1 = tile T - 1's
          // second sub-tile, 2 = tile T + 1's first); this step's fragments were read by the step before it
          const int pr = r > 0 ? r - 1 : R - 1;
          const int nsub = (r > 0 ? sub : sub - 1) + 1;
          const bool even = ((3 * sub + r) & 1) == 0;
          uint32_t(&pin)[8] = even ? P0 : P1;
          uint32_t(&pout)[8] = even ? P1 : P0;
          const u32x4 vf0 = fv0, vf1 = fv1, kf0 = fk0, kf1 = fk1;

          f32x16& sv = s[r];               // S^T of this step; dead after it (the row's next S^T is written one step later)
          if (!fast) {
            const uint32_t kbg = (uint32_t)(kw[r] >> (32 * sub)) >> (4 * g);   // bit c_row(v, g) - 4 g = 8 (v / 4) + v % 4
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const float xv = dead[r] ? 0.f : sv[v];
              sv[v] = (kbg & (1u << (8 * (v >> 2) + (v & 3)))) ? xv : -INFINITY;
            }
          }
          uint32_t pk[8];
          softmax_step(sv, pk, la[r][0], la[r][1]);
          // the sums are taken in this step, between its MFMAs (left free, the compiler sinks every step's v_dot2 to the end
          // of the tile: 40 more live registers and a VALU burst the matrix core cannot overlap)
          asm volatile("" : "+v"(la[r][0]), "+v"(la[r][1]));
          o[pr] =mfma32(as_bf8(vf0), as_bf8(u32x4{pin[0], pin[1], pin[2], pin[3]}), o[pr]);
          o[pr] = mfma32(as_bf8(vf1), as_bf8(u32x4{pin[4], pin[5], pin[6], pin[7]}), o[pr]);
          s[pr] = qk(kf0, kf1, pr, (nsub & 1) ? bq[1] : bq[0]);
          // the next step's fragments: (sub, r + 1), else (1, 0), else tile T + 1's (0, 0) (V^T of this tile's second
          // sub-tile, K of tile T + 1's first: published by this tile's barrier)
          if (r + 1 < R) frags(bt, sub, sub == 0 ? bt : bn, sub == 0 ? 1 : 0, r);
          else if (sub == 0) frags(bt, 0, bt, 1, R - 1);
          else frags(bt, 1, bn, 0, R - 1);
          // one MFMA every few softmax instructions, so neither unit waits on the other
          __builtin_amdgcn_sched_group_barrier(0x402, 8, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x402, 6, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
          __builtin_amdgcn_sched_group_barrier(0x402, 6, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x402, 6, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) pout[jj] = pk[jj];
        }
      }
    };

    for (int T = 0; T < nT; ++T) {
      const int bn = bt == TA_NB - 1 ? 0 : bt + 1;
      const int bp = bn == TA_NB - 1 ? 0 : bn + 1;     // (T + 2) mod 3 = (T - 1) mod 3
      uint64_t kw[R];
      bool fast;
      if (!MASKED || all_full) {
#pragma unroll
        for (int r = 0; r < R; ++r) kw[r] = ~0ull;
        fast = true;
      } else {
        uint64_t kall = ~0ull;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          kw[r] = keep_word(cur, r, T);
          kall &= kw[r];
        }
        fast = kall == ~0ull && !dead_any;
      }
      if (MASKED) tile(fast, T, bp, bn, kw);
      else tile(true, T, bp, bn, kw);
      bt = bn;
    }

    // ---- item end: the last step's P.V (row R - 1 of the last sub-tile, with P0 and the V^T fragments the last step read
    // ahead), the flag, and the normalised output through the wave's LDS staging rows as contiguous 16-byte stores.
    // Reference 0 is exact for a query whose row sum lies in [2^-32, 2^64): no exp2 overflowed (every term is below the
    // sum), and the largest term is at least 2^-45 (S <= 2^13 terms), so the terms that underflowed weigh below 2^-80 of
    // it.  A query outside that range (or not finite) sends the work item to the fallback kernel.
    o[R - 1] = mfma32(as_bf8(fv0), as_bf8(u32x4{P0[0], P0[1], P0[2], P0[3]}), o[R - 1]);
    o[R - 1] = mfma32(as_bf8(fv1), as_bf8(u32x4{P0[4], P0[5], P0[6], P0[7]}), o[R - 1]);
    float lt[R];
    bool redo = false;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      lt[r] = half_sum(la[r][0] + la[r][1]);
      redo |= __builtin_amdgcn_ballot_w64(r < cur.nrow && cur.q < Sv && !(lt[r] >= TD_PS_MIN && lt[r] < TD_PS_MAX)) != 0;
    }
    uint64_t oa[6] = {FPF_KARG(redo), FPF_KARG(out), FPF_KARG(os[0]), FPF_KARG(os[1]), FPF_KARG(os[2]), FPF_KARG(os[3])};
    karg_wait(oa);
    // this item's output rows (row i0 of (b, h)); every wave writes its flag (no clearing needed)
    uint16_t* const obase = reinterpret_cast<uint16_t*>(oa[1]) + cur.b * (int64_t)oa[2] + cur.i0 * (int64_t)oa[3] + cur.h * (int64_t)oa[4];
    if (l == 0) reinterpret_cast<uint32_t*>(oa[0])[(size_t)w * NW + wave] = redo;
    if (!redo && NW == 4) {                                  // a flagged item is recomputed whole by the fallback kernel
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (r >= cur.nrow || cur.q >= Sv) continue;
        const float inv = lt[r] > 0.f ? 1.0f / lt[r] : 0.f;
        uint16_t* op = obase + r * (int64_t)oa[3] + cur.q * (int64_t)oa[5];
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const int d0 = 8 * qd + 4 * g;
          *reinterpret_cast<u32x2*>(op + d0) =
              u32x2{pack2(o[r][4 * qd] * inv, o[r][4 * qd + 1] * inv), pack2(o[r][4 * qd + 2] * inv, o[r][4 * qd + 3] * inv)};
        }
      }
    } else if (!redo) {
      uint16_t* so = &sO[wave][0];
      const int64_t qbase = (int64_t)cur.q - n;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (r >= cur.nrow) continue;
        const float inv = lt[r] > 0.f ? 1.0f / lt[r] : 0.f;
        rt_wave_lds_sync();                                 // the previous row's reads of the staging rows are done
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const int d0 = 8 * qd + 4 * g;
          *reinterpret_cast<u32x2*>(so + n * TA_OP + d0) =
              u32x2{pack2(o[r][4 * qd] * inv, o[r][4 * qd + 1] * inv), pack2(o[r][4 * qd + 2] * inv, o[r][4 * qd + 3] * inv)};
        }
        rt_wave_lds_sync();
        uint16_t* ob = obase + r * (int64_t)oa[3];
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int qq = 16 * half + (l >> 2), cc = 8 * (l & 3);            // lane: query qq, d cc .. cc + 7
          const u32x4 v = *reinterpret_cast<const u32x4*>(so + qq * TA_OP + cc);
          if (qbase + qq < Sv) *reinterpret_cast<u32x4*>(ob + (qbase + qq) * TA_D + cc) = v;   // out rows: 32 contiguous
        }
      }
    }
    cur = nxt;
    item_of(w + 2 * nwg < hi ? w + 2 * nwg : (w + nwg < hi ? w + nwg : w), nxt);
  }
  vm_wait<0>();                                         // no DMA may land after the wave ends
}

// ---------------------------------------------------------------------------------------------------------------- fallback core
// The work items the fast kernel flagged (a query whose reference-0 row sum lies outside [2^-32, 2^64)), recomputed whole
// with the same operands and work split in two passes over the keys: the first repeats the fast kernel's row sums
// (reference 0, the same MFMA / exp2 / bf16 / dot2 sequence) and takes each query's max; the second computes O and l with
// reference 0 for the queries whose sum is in range -- the fast kernel's bits, whichever kernel finishes them -- and the
// query's max for the others.  One step per (row, 32-key sub-tile), the keep bits built in LDS from the mask, K / V^T
// tiles by DMA through the same three-buffer ring.  A workgroup reads the flags of 64 of its items at a time and skips
// the unflagged ones.
template <int NW, bool VROWS>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2))) triattn_core_bf16_redo(const CoreParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t sK[TA_NB][TA_R][TA_KT * TA_D];
  __shared__ __attribute__((aligned(16))) uint16_t sV[TA_NB][TA_R][TA_D * TA_KT];
  __shared__ uint64_t sKeepAll[TA_R][TA_MAXW];
  __shared__ int sAlive[TA_R];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, n = l & 31, g = l >> 5;
  // the host checks that the grid fits 31 bits: the workgroup decode is 32-bit
  const uint32_t nq = (uint32_t)cdiv(p.S, 32 * NW), nr = (uint32_t)cdiv(p.N, TA_R), H = (uint32_t)p.H;
  const uint32_t total = (uint32_t)p.B * H * nr * nq;
  // the work items of this workgroup are blockIdx.x + k gridDim.x; 64 of them are checked per round (lane l reads item l's
  // flags), and only the flagged ones are recomputed
  for (uint32_t base = blockIdx.x; base < total; base += 64u * gridDim.x) {
  uint64_t need;
  {
    const uint32_t wl = base + (uint32_t)l * gridDim.x;
    uint32_t any = 0;
    if (wl < total) {
#pragma unroll
      for (int v = 0; v < NW; ++v) any |= p.redo[(size_t)wl * NW + v];
    }
    need = __builtin_amdgcn_ballot_w64(any != 0);
  }
  while (need) {
  const uint32_t w = base + (uint32_t)__builtin_ctzll(need) * gridDim.x;
  need &= need - 1;
  __syncthreads();                                 // every wave is done with the previous item's LDS
  const uint32_t qt = w % nq, rg = (w / nq) % nr, bh = w / (nq * nr);
  const int64_t b = bh / H, h = bh % H;
  const int64_t i0 = (int64_t)rg * TA_R;
  const int64_t q = (int64_t)qt * (32 * NW) + wave * 32 + n;
  const bool qlive = q < p.Sv;                     // (Sv <= Sqk: a live query's row is in q)

  bf16x8 qf[TA_R][2];
#pragma unroll
  for (int r = 0; r < TA_R; ++r) {
    const int64_t i = i0 + r;
    const bool ok = i < p.N && qlive;
    const uint16_t* qp = p.q + b * p.qs[0] + (ok ? i : 0) * p.qs[1] + h * p.qs[2] + (ok ? q : 0) * p.qs[3] + 8 * g;
    qf[r][0] = as_bf8(ok ? *reinterpret_cast<const u32x4*>(qp) : u32x4{0, 0, 0, 0});
    qf[r][1] = as_bf8(ok ? *reinterpret_cast<const u32x4*>(qp + 16) : u32x4{0, 0, 0, 0});
  }


  // DMA: chunk block c (1 KB) of each row's K tile (keys 16c .. 16c + 15) and V tile (V rows: keys 16c .. 16c + 15 as for K;
  // V^T: rows 8c .. 8c + 7) is moved by wave c (4 waves: both) or by waves c (K) and 4 + c (V) (8 waves); rows past N read row
  // i0 (never stored).  Row bases are scalar, the in-tile byte offsets per lane are fixed.
  const int wc = wave & 3;
  const uint16_t* kb[TA_R];
  const uint16_t* vb[TA_R];
  uint32_t koff, koffL, voff, voffL;
  {
    const int kk = 16 * wc + (l >> 2), kc = (l & 3) ^ ((kk >> 2) & 3);
    const int64_t kl = p.Sqk - 1 - (p.S - TA_KT);   // the last tile's key rows past Sqk re-read row Sqk - 1 (masked keys)
    koff = (uint32_t)((kk * p.ks[3] + 8 * kc) * 2);
    koffL = (uint32_t)(((kk < kl ? kk : kl) * p.ks[3] + 8 * kc) * 2);
    if constexpr (VROWS) {
      voff = (uint32_t)((kk * p.vs[3] + 8 * kc) * 2);
      voffL = (uint32_t)(((kk < kl ? kk : kl) * p.vs[3] + 8 * kc) * 2);
    } else {
      const int vd = 8 * wc + (l >> 3), vc = (l & 7) ^ ((vd >> 1) & 7);
      voff = voffL = (uint32_t)((vd * p.vs[3] + 8 * vc) * 2);
    }
#pragma unroll
    for (int r = 0; r < TA_R; ++r) {
      const int64_t ii = i0 + r < p.N ? i0 + r : i0;
      kb[r] = p.k + b * p.ks[0] + ii * p.ks[1] + h * p.ks[2];
      vb[r] = p.v + b * p.vs[0] + ii * p.vs[1] + h * p.vs[2];
    }
  }
  // LDS byte addresses of this wave's chunk block in buffer 0, row 0 (buffer / row steps are constants)
  const uint32_t kl0 = lds_addr(&sK[0][0][512 * wc]), vl0 = lds_addr(&sV[0][0][512 * wc]);
  constexpr uint32_t TILE_B = TA_KT * TA_D * 2;
  const bool v_mover = NW > 4 && wave >= 4;
  auto dma_tile = [&](int64_t k0, int buf) {
#pragma unroll
    for (int r = 0; r < TA_R; ++r) {
      if (NW == 4 || !v_mover) lds_dma16_s(k0 + TA_KT == p.S ? koffL : koff, kb[r] + k0 * p.ks[3], kl0 + (uint32_t)(buf * TA_R + r) * TILE_B);
      if (NW == 4 || v_mover)
        lds_dma16_s(k0 + TA_KT == p.S ? voffL : voff, vb[r] + (VROWS ? k0 * p.vs[3] : k0), vl0 + (uint32_t)(buf * TA_R + r) * TILE_B);
    }
  };
  // The wait counts (vm_wait4<DMA_OPS + 4>, vm_wait4<4>) assume exactly DMA_OPS operations per dma_tile and 4 per
  // bias_issue, every one issued unconditionally and in the order of the loop below: a wait that counted fewer operations
  // than were issued after the load it guards would let that load land in registers already reused.
  constexpr int DMA_OPS = (NW == 4 ? 2 : 1) * TA_R;

  // the wave's row of register-order bias blocks (a wave past S reads block row 0, never stored)
  const int64_t qw = q - n < p.S ? (q - n) >> 5 : 0;
  const float* brow = static_cast<const float*>(p.bias) + b * p.bs[0] + h * p.bs[1] + qw * (p.S >> 5) * 1024;
  const uint32_t boff = (uint32_t)l * 16;
  // bias of the key sub-tile starting at kb (keys kb + 8 qd + 4 g + 0..3: D-layout rows of the S^T accumulator): 4 operations
  auto bias_issue = [&](int64_t kb, f32x4 (&dst)[4]) {
    const float* sb = brow + (kb >> 5) * 1024;
    dst[0] = gload4_async<0>(boff, sb);
    dst[1] = gload4_async<1024>(boff, sb);
    dst[2] = gload4_async<2048>(boff, sb);
    dst[3] = gload4_async<3072>(boff, sb);
  };

  // fragment offsets (bf16 elements) inside a row's K / V^T tile
  const int kfo0 = n * TA_D + 8 * ((g) ^ ((n >> 2) & 3));            // key n, chunk g (k-step 0); sub-tile adds 32 keys
  const int kfo1 = n * TA_D + 8 * ((g + 2) ^ ((n >> 2) & 3));        // chunk g + 2 (k-step 1)
  const int vsw = (n >> 1) & 7;
  const uint32_t vo0 = VROWS ? vrows_off(l, 0) : 0u, vo2 = VROWS ? vrows_off(l, 2) : 0u;
  auto qk = [&](const u32x4& k0f, const u32x4& k1f, int r, const f32x4 (&bb)[4]) {
    f32x16 bc;
#pragma unroll
    for (int qd = 0; qd < 4; ++qd)
#pragma unroll
      for (int e = 0; e < 4; ++e) bc[4 * qd + e] = bb[qd][e];
    return mfma32(as_bf8(k1f), qf[r][1], mfma32(as_bf8(k0f), qf[r][0], bc));
  };

  const int64_t nT = p.S / TA_KT;
  // keep words of rows i0 .. i0 + TA_R - 1 from the call's keep table (the fast kernel's, so both kernels mask the same keys);
  // without a table every key is kept.  Rows past N: no key, not dead (never stored)
  const int nw = (int)(p.S >> 6);
  if (wave < TA_R) {
    const int64_t i = i0 + wave;
    const bool rowok = i < p.N;
    const uint64_t* kr = p.keep ? p.keep + (b * p.N + (rowok ? i : 0)) * keep_words(p.S) : nullptr;
    for (int c = l; c < nw; c += 64) sKeepAll[wave][c] = !rowok ? 0ull : kr ? kr[1 + c] : ~0ull;
    if (l == 0) sAlive[wave] = rowok && (!kr || (kr[0] & TK_ALIVE) != 0);
  }
  // the Q and keep-table loads complete here: inside the passes the only vector-memory operations are the counted ones
  vm_wait<0>();
#pragma unroll
  for (int r = 0; r < TA_R; ++r) asm volatile("" : "+v"(qf[r][0]), "+v"(qf[r][1]));
  if (p.qmul != 1.0f) {
#pragma unroll
    for (int r = 0; r < TA_R; ++r) {
      qf[r][0] = as_bf8(scale_bf8(__builtin_bit_cast(u32x4, qf[r][0]), p.qmul));
      qf[r][1] = as_bf8(scale_bf8(__builtin_bit_cast(u32x4, qf[r][1]), p.qmul));
    }
  }
  __syncthreads();
  bool dead[TA_R];
  bool dead_any = false;
#pragma unroll
  for (int r = 0; r < TA_R; ++r) {
    dead[r] = (i0 + r < p.N) && !sAlive[r];
    dead_any |= dead[r];
  }

  f32x16 o[TA_R], s[TA_R];
  float la[TA_R][2], mx[TA_R], ref[TA_R];
  f32x4 bq[2][4];                  // bias of the even / odd sub-tiles
#pragma unroll
  for (int r = 0; r < TA_R; ++r) ref[r] = 0.f;
  for (int pass = 0; pass < 2; ++pass) {
    const bool stats = pass == 0;  // pass 0: row sums and maxima only; pass 1: O and l with the chosen references
#pragma unroll
    for (int r = 0; r < TA_R; ++r) {
      o[r] = f32x16{};
      la[r][0] = la[r][1] = 0.f;
      mx[r] = -INFINITY;
    }
    // issue order DMA(0), bias(0), bias(1), DMA(1) (a one-tile range re-reads tile 0: every operation is issued, so the
    // counts stay exact)
    dma_tile(0, 0);
    bias_issue(0, bq[0]);
    bias_issue(32, bq[1]);
    dma_tile(nT > 1 ? TA_KT : 0, 1);
    vm_wait4<4 + DMA_OPS>(bq[0][0], bq[0][1], bq[0][2], bq[0][3]);  // tile 0 and bias 0 are in (bias 1, tile 1 may be pending)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int r = 0; r < TA_R; ++r) {
      const uint16_t* kt = &sK[0][r][0];
      s[r] = qk(*reinterpret_cast<const u32x4*>(kt + kfo0), *reinterpret_cast<const u32x4*>(kt + kfo1), r, bq[0]);
    }

    int bt = 0;                    // buffer of tile T
    for (int64_t T = 0; T < nT; ++T) {
      const bool moreT = T + 1 < nT;
      const int bn = bt == TA_NB - 1 ? 0 : bt + 1;      // buffer of tile T + 1
      const int bf = bn == TA_NB - 1 ? 0 : bn + 1;      // buffer of tile T + 2: tile T - 1's, free once every wave is past it
      const int64_t k0 = T * TA_KT;
      bias_issue(moreT ? k0 + TA_KT : 0, bq[0]);         // sub-tile 2T + 2 (past the end: a valid re-read, the counts stay exact)
      uint64_t kw[TA_R], kall = ~0ull, kany = 0;
#pragma unroll
      for (int r = 0; r < TA_R; ++r) {
        const uint64_t wv = sKeepAll[r][T];                               // uniform: keep it in scalar registers
        const uint32_t whi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(wv >> 32));
        const uint32_t wlo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)wv);   // unsigned: no sign extension
        kw[r] = ((uint64_t)whi << 32) | (uint64_t)wlo;
        kall &= kw[r];
        kany |= kw[r];
      }
      const bool full = (kall == ~0ull) && !dead_any;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        if (sub == 0) {
          vm_wait4<DMA_OPS + 4>(bq[1][0], bq[1][1], bq[1][2], bq[1][3]);   // bias 2T + 1 (tile T + 1, bias 2T + 2 may be pending)
        } else {
          bias_issue(moreT ? k0 + TA_KT + 32 : 32, bq[1]);                 // sub-tile 2T + 3
          vm_wait4<4>(bq[0][0], bq[0][1], bq[0][2], bq[0][3]);             // bias 2T + 2 and tile T + 1 are in
          __builtin_amdgcn_s_barrier();                                     // every wave's part of tile T + 1 is in, and every
          asm volatile("" ::: "memory");                                    // wave is done with tile T - 1
          dma_tile((T + 2 < nT ? T + 2 : nT - 1) * TA_KT, bf);
        }
        const bool live_sub = (uint32_t)(kany >> (32 * sub)) != 0;
        const bool next = sub == 0 || moreT;                                // the next sub-tile exists
        const uint16_t* knext = sub == 0 ? &sK[bt][0][32 * TA_D] : &sK[bn][0][0];
#pragma unroll
        for (int r = 0; r < TA_R; ++r) {
          // fragment reads first: V^T of this step, K of the row's next S^T
          u32x4 vf0, vf1;
          if constexpr (VROWS) {
            vf0 = vrows_frag(&sV[bt][r][0], 32 * sub, vo0, vo2);
            vf1 = vrows_frag(&sV[bt][r][0], 32 * sub + 16, vo0, vo2);
          } else {
            const uint16_t* vt = &sV[bt][r][n * TA_KT];
            vf0 = *reinterpret_cast<const u32x4*>(vt + 8 * ((4 * sub + g) ^ vsw));
            vf1 = *reinterpret_cast<const u32x4*>(vt + 8 * ((4 * sub + 2 + g) ^ vsw));
          }
          const uint16_t* kt = knext + r * (TA_KT * TA_D);
          u32x4 kf0 = u32x4{0, 0, 0, 0}, kf1 = u32x4{0, 0, 0, 0};
          if (next) {
            kf0 = *reinterpret_cast<const u32x4*>(kt + kfo0);
            kf1 = *reinterpret_cast<const u32x4*>(kt + kfo1);
          }
          if (live_sub) {          // a sub-tile with no kept key in any row adds exact zeros: skipped
            if (!full) {
              const uint32_t kbg = (uint32_t)(kw[r] >> (32 * sub)) >> (4 * g);   // bit c_row(v, g) - 4 g = 8 (v / 4) + v % 4
#pragma unroll
              for (int v = 0; v < 16; ++v) {
                const float sv = dead[r] ? 0.f : s[r][v];
                s[r][v] = (kbg & (1u << (8 * (v >> 2) + (v & 3)))) ? sv : -INFINITY;
              }
            }
            if (stats) {
#pragma unroll
              for (int v = 0; v < 16; ++v) mx[r] = fmaxf(mx[r], s[r][v]);
            } else {
#pragma unroll
              for (int v = 0; v < 16; ++v) s[r][v] -= ref[r];     // ref +0: the values (and bits) are unchanged
            }
            uint32_t pk[8];
            softmax_step(s[r], pk, la[r][0], la[r][1]);
            if (!stats) {
              o[r] = mfma32(as_bf8(vf0), as_bf8(u32x4{pk[0], pk[1], pk[2], pk[3]}), o[r]);
              o[r] = mfma32(as_bf8(vf1), as_bf8(u32x4{pk[4], pk[5], pk[6], pk[7]}), o[r]);
            }
          }
          if (next) s[r] = qk(kf0, kf1, r, sub == 0 ? bq[1] : bq[0]);
        }
      }
      bt = bn;
    }
    vm_wait<0>();                                       // no DMA may land after the pass ends
    __syncthreads();                                    // every wave is done with the tiles before the next pass refills them
    if (stats) {
      // the fast kernel's test on the same sums: in range, reference 0; else the query's max (finite: a live row keeps a
      // key, a dead row's logits are 0)
#pragma unroll
      for (int r = 0; r < TA_R; ++r) {
        const float lt = half_sum(la[r][0] + la[r][1]);
        const float m = half_max(mx[r]);
        ref[r] = ((lt >= TD_PS_MIN && lt < TD_PS_MAX) || !(m > -INFINITY && m < INFINITY)) ? 0.f : m;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < TA_R; ++r) {
    const int64_t i = i0 + r;
    if (i >= p.N || !qlive) continue;
    const float lt = half_sum(la[r][0] + la[r][1]);
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    uint16_t* op = p.out + b * p.os[0] + i * p.os[1] + h * p.os[2] + q * p.os[3];
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const int d0 = 8 * qd + 4 * g;
      *reinterpret_cast<u32x2*>(op + d0) = u32x2{pack2(o[r][4 * qd] * inv, o[r][4 * qd + 1] * inv), pack2(o[r][4 * qd + 2] * inv, o[r][4 * qd + 3] * inv)};
    }
  }
  }
  }
}

// ---------------------------------------------------------------------------------------------------------------- op staging
// The op face (kernels/triattn/__init__.py:1094) hands q, k, v [B, N, H, S, 32] and a [B, 1, H, S, S] bias in its own layout; the
// block-layout core reads q and k in place and wants V^T and the bias as the block's prologue writes them.  One wave per (b, n, h,
// 64-position tile): the tile goes through the wave's LDS rows so each lane stores 32 consecutive positions of one V^T row in the
// core's 16-block key order.
__device__ __forceinline__ int vperm16(int s) { return (s & ~12) | ((s & 4) << 1) | ((s & 8) >> 1); }   // swaps bits 2 and 3

constexpr int ST_VLD = 64 + 8;    // LDS pitch (bf16) of a staged V^T row: 144 B

__global__ void __launch_bounds__(256) triattn_stage_v(const StageParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t sV[4][32 * ST_VLD];
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int64_t tiles = p.Sp / 64, total = p.B * p.N * p.H * tiles;
  const int64_t unit = (int64_t)blockIdx.x * 4 + wave;
  if (unit >= total) return;                                  // whole waves leave: only wave-level synchronisation below
  const int64_t tile = unit % tiles, bnh = unit / tiles, h = bnh % p.H, bn = bnh / p.H, n = bn % p.N, b = bn / p.N;
  // the tile's 64 positions x 64 bytes as 256 16-byte chunks: load i moves chunk l + 64 i (position (l + 64 i) / 4, head-dim chunk
  // l % 4), so each instruction reads 1 KB of the caller's rows when they are contiguous
  const int dc = l & 3;
  uint16_t* sv = sV[wave];
  uint16_t* vdst = p.v2 + ((b * p.N + n) * p.H + h) * 32 * p.Sp + tile * 64;      // V^T row 0 of this tile
  const uint16_t* vb = p.v + b * p.vs[0] + n * p.vs[1] + h * p.vs[2];
  if (!p.v_t) {
    // chunk (position ps, dims 8 dc .. 8 dc + 7) goes to column vperm16(ps) of LDS rows 8 dc .. 8 dc + 7
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ps = (l >> 2) + 16 * i;
      const int64_t s = tile * 64 + ps;
      const u32x4 r = s < p.S ? *reinterpret_cast<const u32x4*>(vb + s * p.vs[3] + 8 * dc) : u32x4{0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sv[(8 * dc + 2 * e) * ST_VLD + vperm16(ps)] = (uint16_t)(r[e] & 0xffff);
        sv[(8 * dc + 2 * e + 1) * ST_VLD + vperm16(ps)] = (uint16_t)(r[e] >> 16);
      }
    }
    rt_wave_lds_sync();
    // V^T tile: 32 rows x 128 bytes; store i moves row (l + 64 i) / 8, chunk l % 8: each instruction writes 8 whole 128-byte row
    // segments
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = (l >> 3) + 8 * i, c = l & 7;
      *reinterpret_cast<u32x4*>(vdst + d * p.Sp + 8 * c) = *reinterpret_cast<const u32x4*>(sv + d * ST_VLD + 8 * c);
    }
  } else {
    // V^T given: row d's 64 keys as 4 blocks of 16; lane (d, block) reads one block, and in it the 8-byte halves 4-7 and 8-11
    // trade places
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int d = (l >> 2) + 16 * i, blk = l & 3;
      const uint16_t* vr = vb + d * p.vs[3];
      const int64_t k0 = tile * 64 + 16 * blk;
      u32x4 c0 = {0, 0, 0, 0}, c1 = {0, 0, 0, 0};
      if (k0 + 16 <= p.S) {
        c0 = *reinterpret_cast<const u32x4*>(vr + k0);
        c1 = *reinterpret_cast<const u32x4*>(vr + k0 + 8);
      } else {
        uint16_t t[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) t[e] = k0 + e < p.S ? vr[k0 + e] : (uint16_t)0;
        c0 = u32x4{t[0] | (uint32_t)t[1] << 16, t[2] | (uint32_t)t[3] << 16, t[4] | (uint32_t)t[5] << 16, t[6] | (uint32_t)t[7] << 16};
        c1 = u32x4{t[8] | (uint32_t)t[9] << 16, t[10] | (uint32_t)t[11] << 16, t[12] | (uint32_t)t[13] << 16, t[14] | (uint32_t)t[15] << 16};
      }
      uint16_t* dst = vdst + d * p.Sp + 16 * blk;
      *reinterpret_cast<u32x4*>(dst) = u32x4{c0[0], c0[1], c1[0], c1[1]};
      *reinterpret_cast<u32x4*>(dst + 8) = u32x4{c0[2], c0[3], c1[2], c1[3]};
    }
  }
}

// bias2 block (qb, kb) of plane (b, h): one wave, piece j = 256 consecutive floats, lane (n, g) = query qb 32 + n, keys kb 32 + 8j +
// 4g .. + 3 (the register order of the core's S^T accumulator); values past S are zero.
__global__ void __launch_bounds__(256) triattn_stage_bias(const StageParams p) {
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63, n = l & 31, g = l >> 5;
  const int64_t nb = p.Sp / 32, total = p.B * p.H * nb * nb;
  const int64_t unit = (int64_t)blockIdx.x * 4 + wave;
  if (unit >= total) return;
  const int64_t kb = unit % nb, qb = (unit / nb) % nb, bh = unit / (nb * nb), h = bh % p.H, b = bh / p.H;
  const int64_t qi = qb * 32 + n;
  const int64_t rowoff = b * p.bs[0] + h * p.bs[1] + (qi < p.S ? qi : 0) * p.bs[2];
  float* dst = p.bias2 + bh * p.Sp * p.Sp + ((qb * nb + kb) << 10) + l * 4;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t key = kb * 32 + 8 * j + 4 * g + e;
      float x = 0.f;
      if (qi < p.S && key < p.S)
        x = p.bias_bf16 ? bf2f(static_cast<const uint16_t*>(p.bias)[rowoff + key]) : static_cast<const float*>(p.bias)[rowoff + key];
      w[e] = x * LOG2E;
    }
    *reinterpret_cast<f32x4*>(dst + 256 * j) = w;
  }
}

// ---------------------------------------------------------------------------------------------------------------- launchers
int keep_table_launch(const void* mask, int mask_f32, const int64_t ms[3], int64_t B, int64_t N, int64_t S, int64_t Sv, uint64_t* keep,
                      hipStream_t st, char* err, size_t errlen, bool dry) {
  if (!keep) return fail(err, errlen, FPF_E_ARGS, "keep table: table is NULL");
  if (S % TA_KT != 0 || S > (int64_t)TA_KT * TA_MAXW) return fail(err, errlen, FPF_E_SHAPE, "keep table: S a multiple of 64 up to %d", TA_KT * TA_MAXW);
  if (Sv <= 0 || Sv > S) return fail(err, errlen, FPF_E_SHAPE, "keep table: real keys %lld outside (0, %lld]", (long long)Sv, (long long)S);
  const int64_t blocks = cdiv(B * N, 4);
  if (blocks > 0x7fffffffLL) return fail(err, errlen, FPF_E_SHAPE, "keep table: grid too large");
  if (dry) return FPF_OK;
  if (mask && !mask_f32 && ms[2] == 1 && aligned16(mask) && ms[0] % 16 == 0 && ms[1] % 16 == 0 && Sv % 16 == 0) {
    hipLaunchKernelGGL(triattn_keep_bits_u8, dim3((unsigned)blocks), dim3(256), 0, st, static_cast<const uint8_t*>(mask), ms[0], ms[1], B, N, S, Sv, keep);
    return launched(err, errlen, "triattn_keep_bits_u8");
  }
  hipLaunchKernelGGL(triattn_keep_bits, dim3((unsigned)blocks), dim3(256), 0, st, mask, mask_f32, ms[0], ms[1], ms[2], B, N, S, Sv, keep);
  return launched(err, errlen, "triattn_keep_bits");
}

// The caller has checked the layout: S a multiple of 64 up to 64 TA_MAXW, fp32 bias with 16-byte aligned rows, q / k / V^T
// 16-byte aligned with strides in multiples of 8, out rows of 32 contiguous, 16-byte aligned bf16 (out stride[3] = 32,
// others multiples of 8), scale 1, p.redo holding redo_words(B, N, H, S) words.  8 waves (256 queries)
// share each K / V^T tile where S fills whole 256-query tiles and the grid still has 8 or more workgroups per CU; 4 waves (128
// queries) elsewhere.  The fallback runs on the same stream right after the fast kernel, over the same grid.
// The block-layout core's per-lane byte offsets from its scalar bases are 32-bit: q (query, d), K (key row of a tile, and the
// tile's offset from tile 0), V^T (d row), and a row's from the item's first row.
bool pipe_offsets_fit(int64_t S, const int64_t* qs, const int64_t* ks, const int64_t* vs, bool v_rows) {
  const int64_t lim = 0x7fffffffLL;
  return qs[3] >= 0 && ks[3] >= 0 && vs[3] >= 0 && qs[1] >= 0 && ks[1] >= 0 && vs[1] >= 0 && S <= lim &&
         (S - 1) * qs[3] * 2 + 64 <= lim && S * ks[3] * 2 <= lim && (v_rows ? S : TA_D) * vs[3] * 2 <= lim &&
         (TA_R - 1) * std::max(qs[1], std::max(ks[1], vs[1])) * 2 <= lim;
}

int pipe_core_launch(const CoreParams& p, hipStream_t st, char* err, size_t errlen, bool dry) {
  const int64_t rows_heads = p.B * p.H * cdiv(p.N, TA_R);
  // 8 waves share each K / V^T tile among 256 queries; where S is not a multiple of 256 the last query tile is partly padding.
  // A query slot of the 8-wave split costs about 95 % of one of the 4-wave split (items of 128 queries per 4 waves): the
  // 8-wave split is taken when its slots at that rate cost less, and the grid holds 8 or more workgroups per CU (measured,
  // op / block at the starting node: S = 768 8-wave 0.447 / 0.603 ms against 0.473 / 0.622; S = 800 (832 padded) 4-wave
  // 0.692 / 0.783 against 0.710 / 0.813; S = 640 4-wave 0.297 / 0.426 against 0.326 / 0.447; S = 384 8-wave 11-15 % slower)
  const int64_t q8 = cdiv(p.S, 32 * TA_DMA_WAVES), q4 = cdiv(p.S, 128);
  const bool wide = 19 * q8 * (32 * TA_DMA_WAVES) < 20 * q4 * 128 && rows_heads * q8 >= 8 * (int64_t)num_cus();
  const int64_t total = wide ? rows_heads * q8 : rows_heads * q4;
  if (cdiv(total, 8) * 8 > 0x7fffffffLL) return fail(err, errlen, FPF_E_SHAPE, "grid too large");
  if (p.bs[2] < 0 || !pipe_offsets_fit(p.S, p.qs, p.ks, p.vs, p.v_rows != 0) || p.B * p.N > 0x7fffffffLL)
    return fail(err, errlen, FPF_E_SHAPE, "v_layout 2 / 3: q / bias / k / v in-item offsets must fit 31 bits");
  if (p.Sv <= 0 || p.Sv > p.S || (p.Sv < p.S && !p.keep))
    return fail(err, errlen, FPF_E_ARGS, "v_layout 2 / 3: %lld real keys of %lld need a keep table masking the padding", (long long)p.Sv, (long long)p.S);
  if (dry) return FPF_OK;
  // persistent grids: one fast workgroup per CU walking every nwg-th item of its XCD's range (two per CU for the 4-wave
  // split, whose LDS and registers fit twice), and at least 8 workgroups, so that every XCD's range has one (with fewer
  // than 8 items some of them have none to do); the fallback scans its share of the flags
  const dim3 grid((unsigned)std::max<int64_t>(8, std::min<int64_t>(total, (wide ? 1 : 2) * (int64_t)num_cus())));
  const dim3 redo_grid((unsigned)std::min<int64_t>(total, num_cus()));
  if (p.v_rows) {
    if (wide) {
      if (p.keep) hipLaunchKernelGGL((triattn_core_bf16_pipe<TA_DMA_WAVES, true, true>), grid, dim3(64 * TA_DMA_WAVES), 0, st, p);
      else hipLaunchKernelGGL((triattn_core_bf16_pipe<TA_DMA_WAVES, false, true>), grid, dim3(64 * TA_DMA_WAVES), 0, st, p);
      hipLaunchKernelGGL((triattn_core_bf16_redo<TA_DMA_WAVES, true>), redo_grid, dim3(64 * TA_DMA_WAVES), 0, st, p);
    } else {
      if (p.keep) hipLaunchKernelGGL((triattn_core_bf16_pipe<4, true, true>), grid, dim3(256), 0, st, p);
      else hipLaunchKernelGGL((triattn_core_bf16_pipe<4, false, true>), grid, dim3(256), 0, st, p);
      hipLaunchKernelGGL((triattn_core_bf16_redo<4, true>), redo_grid, dim3(256), 0, st, p);
    }
  } else if (wide) {
    if (p.keep) hipLaunchKernelGGL((triattn_core_bf16_pipe<TA_DMA_WAVES, true, false>), grid, dim3(64 * TA_DMA_WAVES), 0, st, p);
    else hipLaunchKernelGGL((triattn_core_bf16_pipe<TA_DMA_WAVES, false, false>), grid, dim3(64 * TA_DMA_WAVES), 0, st, p);
    hipLaunchKernelGGL((triattn_core_bf16_redo<TA_DMA_WAVES, false>), redo_grid, dim3(64 * TA_DMA_WAVES), 0, st, p);
  } else {
    if (p.keep) hipLaunchKernelGGL((triattn_core_bf16_pipe<4, true, false>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((triattn_core_bf16_pipe<4, false, false>), grid, dim3(256), 0, st, p);
    hipLaunchKernelGGL((triattn_core_bf16_redo<4, false>), redo_grid, dim3(256), 0, st, p);
  }
  return launched(err, errlen, "triattn_core_bf16_pipe");
}

int op_stage_launch(const StageParams& p, hipStream_t st, char* err, size_t errlen, bool dry) {
  if (p.Sp % 64 || p.Sp < p.S || p.S <= 0) return fail(err, errlen, FPF_E_SHAPE, "staging: Sp %lld for S %lld", (long long)p.Sp, (long long)p.S);
  const int64_t u1 = p.B * p.N * p.H * (p.Sp / 64), u2 = p.B * p.H * (p.Sp / 32) * (p.Sp / 32);
  if (cdiv(u1, 4) > 0x7fffffffLL || cdiv(u2, 4) > 0x7fffffffLL) return fail(err, errlen, FPF_E_SHAPE, "staging: grid too large");
  if (dry) return FPF_OK;
  if (p.v2) hipLaunchKernelGGL(triattn_stage_v, dim3((unsigned)cdiv(u1, 4)), dim3(256), 0, st, p);
  hipLaunchKernelGGL(triattn_stage_bias, dim3((unsigned)cdiv(u2, 4)), dim3(256), 0, st, p);
  return launched(err, errlen, "triattn_stage_v / triattn_stage_bias");
}

}  // namespace fpf
