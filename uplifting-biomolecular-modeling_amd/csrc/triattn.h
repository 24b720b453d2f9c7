// Definitions shared by the triangle-attention kernels (triattn.hip: the op core, the fused block's stages; triattn_pipe.hip:
// the block-layout core and its keep-bit table).
#pragma once
#include "rowtile.h"

namespace fpf {

constexpr int TA_D = 32;
constexpr int TA_R = 3;          // pair rows per workgroup sharing the bias tile (3: the register budget of 2 waves / SIMD)
constexpr int TA_KT = 64;        // keys per staged tile (two MFMA sub-tiles of 32)
constexpr int TA_KLD = 40;       // LDS pitch (bf16) of a K row: 80 B, conflict-free 16-byte reads
constexpr int TA_VLD = 68;       // LDS pitch (bf16) of a V^T row: 136 B, conflict-free 8-byte reads
constexpr int TA_MAXW = 128;     // block-layout core: keep-bit words per row held in LDS (S <= 8192)
constexpr float LOG2E = 1.4426950408889634f;
constexpr float TA_HEADROOM = 8.0f;   // log2 units the running max may lag the true one before O and l are rescaled
static_assert(TA_R <= 4, "one wave computes the keep bits of one staged row");

struct CoreParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t qs[5], ks[5], vs[5];   // v_t = 0: vs = [b, n, h, key, d] strides; v_t = 1: [b, n, h, d, key] (V stored transposed)
  int v_t;
  const void* bias;
  int bias_bf16;
  int bias_vec;                  // fp32 bias whose rows start 16-byte aligned: float4 loads
  int64_t bs[4];
  const void* mask;
  int mask_f32;
  int64_t ms[3];
  uint16_t* out;
  int64_t os[5];
  int64_t B, N, H, S;
  float scale;
  const uint64_t* keep;          // block-layout core: keep table [B, N, keep_words(S)] of the mask, or NULL (every key kept)
  uint32_t* redo;                // block-layout core: one flag per (work item, wave), written by the fast kernel
  int64_t Sv;                    // block-layout core: the real keys / queries (<= S); keys Sv .. S - 1 pad the key axis to a
                                 // multiple of 64 and are masked by the keep table, queries past Sv are never stored
  int64_t Sqk;                   // block-layout core: the query / key rows q and k hold (S - 64 < Sqk <= S); queries past it read
                                 // query 0 (never stored), the last K tile's rows past it re-read row Sqk - 1 (keys the keep
                                 // table masks)
  float qmul;                    // block-layout core: the factor q is multiplied by in registers, each product rounded to bf16
                                 // once (1: q comes already multiplied)
  int v_rows;                    // block-layout core: V as key rows [b, n, h, key, d] (vs its strides; the last tile's rows past
                                 // Sqk re-read row Sqk - 1, like K), else V^T [b, n, h, d, key] with keys in the 16-block order
};

__device__ __forceinline__ bool mask_keep(const CoreParams& p, int64_t b, int64_t i, int64_t key) {
  if (!p.mask) return true;
  const int64_t o = b * p.ms[0] + i * p.ms[1] + key * p.ms[2];
  return p.mask_f32 ? (static_cast<const float*>(p.mask)[o] != 0.0f) : (static_cast<const uint8_t*>(p.mask)[o] != 0);
}

__device__ __forceinline__ float bias_at(const CoreParams& p, int64_t off) {
  return p.bias_bf16 ? bf2f(static_cast<const uint16_t*>(p.bias)[off]) : static_cast<const float*>(p.bias)[off];
}

// eight bf16 of q times m, each product rounded to bf16 once (the op face's staging and the block-layout core's in-register
// scaling compute the same bits)
__device__ __forceinline__ u32x4 scale_bf8(const u32x4& x, float m) {
  u32x4 w;
#pragma unroll
  for (int e = 0; e < 4; ++e) w[e] = pack2(lo_bf(x[e]) * m, hi_bf(x[e]) * m);
  return w;
}

// V of the block-layout core as key rows (v_rows): a 64-key tile in LDS holds key k's 32 values as four 16-byte chunks, chunk c
// at position c ^ ((k >> 2) & 3), as the K tile does.  The P.V product's A operand -- lane (n, g): d = n and the keys
// kb + 4 g + 0..3, kb + 8 + 4 g + 0..3 of a 16-key step -- comes from two ds_read_b64_tr_b16: within each group of 16 lanes,
// lane 4 e + q reads 4 values (d0 + 4 q .. + 3) of key row k0 + e, and lane j receives the values of d0 + j in rows
// k0 .. k0 + 3.  vrows_off: lane l's byte offset in a tile for the read at key base 0 (S2 = 0) or 8 (S2 = 2) of a step.
__device__ __forceinline__ uint32_t vrows_off(int l, int S2) {
  const int h16 = l >> 4, il = l & 15, e = il >> 2, q = il & 3, g = h16 >> 1;
  const int c = 2 * (h16 & 1) + (q >> 1);
  return (uint32_t)((4 * g + e) * 64 + (c ^ (g + S2)) * 16 + (q & 1) * 8);
}
typedef short v4i16_t __attribute__((ext_vector_type(4)));
// the A-operand fragment of the 16-key step starting at key kb (a multiple of 16) of a V-rows tile
__device__ __forceinline__ u32x4 vrows_frag(const uint16_t* tile, int kb, uint32_t vo0, uint32_t vo2) {
  typedef __attribute__((address_space(3))) v4i16_t lds_v4;
  char* t = const_cast<char*>(reinterpret_cast<const char*>(tile));
  const v4i16_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4*)(t + kb * 64 + vo0));
  const v4i16_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4*)(t + (kb + 8) * 64 + vo2));
  const u32x2 a2 = __builtin_bit_cast(u32x2, a), b2 = __builtin_bit_cast(u32x2, b);
  return u32x4{a2[0], a2[1], b2[0], b2[1]};
}

// Bias plane of the block-layout core (v_layout 2): S x S fp32 (query q, key k) in 32 x 32 blocks, block (q / 32, k / 32) at
// element ((q / 32) (S / 32) + k / 32) 1024, each block in the order one wave's S^T accumulator holds it -- piece j (keys
// 8 j .. 8 j + 7) of 256 elements, lane n + 32 g (query n, keys 8 j + 4 g .. + 3) 4 elements each -- so a wave loads a
// 32 x 32 sub-tile with four contiguous 1 KB reads.
__host__ __device__ inline int64_t bias_blk_off(int64_t S, int64_t q, int64_t k) {
  return (((q >> 5) * (S >> 5) + (k >> 5)) << 10) + (((k >> 3) & 3) << 8) + (((q & 31) + (((k >> 2) & 1) << 5)) << 2) + (k & 3);
}
constexpr int TA_NB = 3;                                 // K / V^T tile buffers of the block-layout core
constexpr int TA_DMA_WAVES = 8;                          // waves (32 queries each) per workgroup of the block-layout core:
                                                         // 8 share each K / V^T tile among 256 queries (4 move K, 4 V^T)
constexpr float TD_PS_MAX = 18446744073709551616.0f;     // 2^64: a sub-tile's partial row sum at or above it needs a reference
constexpr float TD_PS_MIN = 2.3283064365386963e-10f;     // 2^-32: so does a query's first sub-tile with a kept key summing below it

// 16 bytes at sbase + voff + IMM (scalar base, 32-bit per-lane byte offset) into registers, not waited for here
template <int IMM>
__device__ __forceinline__ f32x4 gload4_async(uint32_t voff, const void* sbase) {
  f32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, %2 offset:%3" : "=v"(v) : "v"(voff), "s"(sbase), "n"(IMM));
  return v;
}
// The same load into registers that hold a live value until now ("+v": the previous value is an input), so the compiler
// keeps that value in place up to the load instead of reusing its registers -- e.g. as the accumulator of an MFMA that reads
// it last
template <int IMM>
__device__ __forceinline__ void gload4_into(f32x4& v, uint32_t voff, const void* sbase) {
  asm volatile("global_load_dwordx4 %0, %1, %2 offset:%3" : "+v"(v) : "v"(voff), "s"(sbase), "n"(IMM));
}
// v_mfma_f32_32x32x16_bf16 into a new tuple (D and C distinct, no copy of C): the compiler's own selection copies C into
// the accumulator when C stays live in other blocks.  Only a following MFMA accumulating onto the result may read it
// next (the same instruction reading its exact D as C needs no wait states; nothing else reads it without the compiler
// seeing an MFMA producer).
__device__ __forceinline__ f32x16 mfma32_new(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  f32x16 d;
  asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %3" : "=&v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}
// One softmax step of the block-layout core (both of its kernels, so they produce the same bits): exp2 of the 16 logits,
// packed to the bf16 pairs the P.V MFMA consumes, and those bf16 values added to the row's two running sums (even pairs
// into a0, odd into a1, in order; v_dot2_f32_bf16 against (1, 1)).  The sums hold exactly the weights O accumulates, so
// each query's weights sum to 1 after the normalisation (summing the unrounded fp32 terms with v_add_f32 is cheaper
// but measurably less accurate at block level).  Every exp2 is issued before the first pack reads one.
__device__ __forceinline__ void softmax_step(const f32x16& sv, uint32_t (&pk)[8], float& a0, float& a1) {
  float e[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) e[v] = fast_exp2(sv[v]);
#pragma unroll
  for (int v = 0; v < 16; v += 2) pk[v >> 1] = pack2(e[v], e[v + 1]);
#pragma unroll
  for (int jj = 0; jj < 8; jj += 2) {
    a0 = dot2_bf16(pk[jj], a0);
    a1 = dot2_bf16(pk[jj + 1], a1);
  }
}
// 8 bytes at a wave-uniform address through the scalar cache, waited for here (lgkmcnt also covers this wave's LDS reads)
__device__ __forceinline__ uint64_t sload64(const uint64_t* a) {
  uint64_t v;
  asm volatile("s_load_dwordx2 %0, %1, 0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(a) : "memory");
  return v;
}
// Fields of the CoreParams block of a kernel whose only argument it is (it starts the kernarg segment), reloaded through the
// scalar cache where they are used, so that a loop running for the whole kernel holds none of them in registers.  Issue the
// loads of one place with karg_issue, then pass every result through karg_wait before the first use.
template <int OFF>
__device__ __forceinline__ uint64_t karg_issue() {
  uint64_t v;
  asm volatile("s_load_dwordx2 %0, %1, %2" : "=s"(v) : "s"(__builtin_amdgcn_kernarg_segment_ptr()), "n"(OFF));
  return v;
}
template <int K>
__device__ __forceinline__ void karg_wait(uint64_t (&v)[K]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < K; ++i) asm volatile("" : "+s"(v[i]));
}
#define FPF_KARG(field) ::fpf::karg_issue<(int)offsetof(::fpf::CoreParams, field)>()
static_assert(offsetof(CoreParams, qmul) + 8 <= sizeof(CoreParams), "a reload of qmul reads 8 bytes inside the block");
// waits until at most N vector-memory operations of this wave are outstanding; the registers of the sub-tile's bias pass
// through the statement so nothing reads them earlier
template <int N>
__device__ __forceinline__ void vm_wait4(f32x4& a, f32x4& b, f32x4& c, f32x4& d) {
  asm volatile("s_waitcnt vmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "n"(N));
}
template <int N>
__device__ __forceinline__ void vm_wait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// The block-layout core (v_layout 2) and its keep table (triattn_pipe.hip).  Keep table of a call: for each (b, attention row
// i) keep_words(S) = S / 64 + 1 words: word 0 = row flags (TK_ALIVE: some key kept, TK_FULL: every one of the S keys kept),
// word 1 + T = the keep bits of keys 64 T .. 64 T + 63 (bit k = key 64 T + k).  Keys at or past Sv (the padding of the key
// axis to a multiple of 64) have bit 0 in every row; a row with no kept key has the bits of all Sv real keys set (it attends
// uniformly to them).
constexpr uint64_t TK_ALIVE = 1, TK_FULL = 2;
__host__ __device__ inline int64_t keep_words(int64_t S) { return S / 64 + 1; }
// Redo flags of a call (one 32-bit word per work item and wave), enough for either split: B H ceil(N / TA_R) times the larger of
// ceil(S / 128) 4 (4 waves of 32 queries per item) and ceil(S / 256) 8 (8 waves; larger when S is an odd multiple of 64 ... 128
// past a multiple of 256).
inline int64_t redo_words(int64_t B, int64_t N, int64_t H, int64_t S) {
  return B * H * cdiv(N, TA_R) * std::max<int64_t>(cdiv(S, 128) * 4, cdiv(S, 256) * 8);
}
// dry = true: every check of the launch, nothing launched (callers that must refuse before their first launch)
// mask NULL: every real key kept (a table that only masks the padding keys Sv .. S - 1)
int keep_table_launch(const void* mask, int mask_f32, const int64_t ms[3], int64_t B, int64_t N, int64_t S, int64_t Sv, uint64_t* keep,
                      hipStream_t st, char* err, size_t errlen, bool dry = false);
bool pipe_offsets_fit(int64_t S, const int64_t* qs, const int64_t* ks, const int64_t* vs, bool v_rows);
int pipe_core_launch(const CoreParams& p, hipStream_t st, char* err, size_t errlen, bool dry = false);

// N a multiple of 64, or any N from 128, up to 8192: the J axis of q / k / V^T / o and of the bias planes is padded to Np = N
// rounded up to 64 (block_np), the padding keys masked by the keep table, the padding queries never stored.  Below 128 keys a
// padded call keeps the op core: with few keys the extra bf16 rounding of q * scale * log2(e) no longer averages out (N = 97
// measured rel-L2 5.0e-3 on the block core against the 5e-3 bar).
inline bool block_layout2(int dtype, int64_t N) {
  return dtype == FPF_DT_BF16 && cdiv(N, TA_KT) * TA_KT <= 64 * TA_MAXW && (N % TA_KT == 0 || N >= 2 * TA_KT);
}
inline int64_t block_np(int dtype, int64_t N) { return block_layout2(dtype, N) ? cdiv(N, TA_KT) * TA_KT : N; }

// The op face's V and bias restaged into the block-layout core's layout (triattn_pipe.hip): v2 = V^T [B, N, H, 32, Sp] with each
// 16-key block in the order 0-3, 8-11, 4-7, 12-15, bias2 = bias * log2(e) as [B, H, Sp, Sp] in 32 x 32 register-order blocks
// (bias_blk_off), Sp = S rounded up to 64, every padding element zero (q and k the core reads in place).  v is read as
// [B, N, H, S, 32] (v_t = 0) or transposed as [B, N, H, 32, S] (v_t = 1); v2 NULL: V is not copied (the core reads its key
// rows in place).  The caller has checked: head_dim rows of 32 contiguous, 16-byte aligned bf16 (strides multiples of 8
// elements).
struct StageParams {
  const uint16_t* v;
  int64_t vs[4];                 // strides of b, n, h, s (v_t = 1: of b, n, h, d)
  int v_t;
  const void* bias;
  int bias_bf16;
  int64_t bs[3];                 // strides of b, h, query (the key stride is 1)
  uint16_t* v2;
  float* bias2;
  int64_t B, N, H, S, Sp;
};
int op_stage_launch(const StageParams& p, hipStream_t st, char* err, size_t errlen, bool dry = false);

}  // namespace fpf
