/* fpf_hip.h -- the C ABI of libfpf_hip.so: the FlashPairformer pair-stack hot path (triangle attention, triangle
 * multiplication, LayerNorm + SwiGLU transition, standalone LayerNorm) as hand-written gfx950 (MI355X) HIP kernels.
 *
 * Every entry point takes one POD argument block whose first field is abi_version (= FPF_ABI_VERSION), a HIP stream
 * (hipStream_t passed as void*, NULL = the null stream) and an error buffer.  Rules shared by all entry points:
 *   - return FPF_OK (0) once the kernels are enqueued; any other value means NOTHING was launched and err holds one line
 *     (the caller's face maps it to a refusal by name);
 *   - every pointer is a caller-owned device pointer (workspaces included); the library allocates and frees nothing and
 *     never synchronises the host, so calls are capture-safe and reentrant across host threads and streams;
 *   - shapes are 64-bit; strides are in ELEMENTS;
 *   - dtype codes: FPF_DT_BF16 = bf16 storage with fp32 accumulation and softmax (the "fast" tier), FPF_DT_F32 = fp32
 *     storage and fp32 arithmetic throughout (the "exact" tier), FPF_DT_F32Z_BF16 (the triangle multiplication only) = fp32
 *     z and out with bf16 operands: the reference's f32z_bf16 class (kernels/trimul/__init__.py:219, an fp32 pair tensor
 *     under bf16 autocast), whose fused rows read z rounded once to bf16 (compute_input, :1248).
 *
 * The reference interface each entry point replaces is cited on its declaration (paths under the reference tree).
 */
#ifndef FPF_HIP_H
#define FPF_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FPF_ABI_VERSION 13  /* 3: v_layout 2 logits in log2 units; fpf_apb_fwd, fpf_apb_bias_fwd; 4: block mask_frame;
                               5: gate / output projection biases b_g, b_o on the tri-att block and its stages;
                               6: the v_layout 2 core reads the mask as a keep-bit table and takes a workspace
                                  (FpfTriattnArgs.keep / workspace / workspace_bytes, fpf_triattn_workspace_bytes);
                               7: the v_layout 2 core's bias (and fpf_triattn_bias_fwd's output for such N) in 32 x 32
                                  register-order blocks;
                               8: the trimul rows mode (FpfTrimulArgs.row0 / rows / fixed_in, fpf_trimul_fixed_fwd,
                                  fpf_trimul_fixed_bytes, fpf_trimul_rows_workspace_bytes);
                               9: FPF_DT_F32Z_BF16 for the trimul (fp32 z / out, bf16 operands and planes);
                               10: the bf16 block runs the v_layout 2 core for every N up to 8192 (its J axis padded to 64:
                                   fpf_triattn_bias_bytes sizes fpf_triattn_bias_fwd's output); fpf_triattn_stage_bytes and the
                                   staged route of fpf_triattn_fwd onto that core;
                               11: x_ln (the caller's own LayerNorm output, ln="stock") appended to FpfTriattnBlockArgs,
                                   FpfTriattnPrologueArgs and FpfTransitionArgs;
                               12: the single track's pair bias projected from the transition's written rows (FpfTransitionArgs
                                   w_z .. z_bias_ld);
                               13: v_layout 3 (the block-layout core reading V as key rows); the op face's staged route reads
                                   q, k and v in place */

enum { FPF_DT_BF16 = 1, FPF_DT_F32 = 2, FPF_DT_U8 = 3, FPF_DT_F32Z_BF16 = 4 };
enum {
  FPF_OK = 0,
  FPF_E_VERSION = 1,   /* abi_version mismatch */
  FPF_E_ARGS = 2,      /* NULL pointer / bad flag */
  FPF_E_SHAPE = 3,     /* a shape this entry point does not serve (e.g. head_dim != 32 on the bf16 core) */
  FPF_E_DTYPE = 4,     /* a dtype code this entry point does not serve */
  FPF_E_ALIGN = 5,     /* a pointer or stride that breaks the 16-byte vector access the kernels use */
  FPF_E_WORKSPACE = 6, /* workspace missing or smaller than the *_workspace_bytes query */
  FPF_E_LAUNCH = 7     /* hipLaunchKernel reported an error (the message carries hipGetErrorString) */
};

/* Library identity.  No counterpart in the reference (its sealed packages carry the same facts in manifests). */
int fpf_abi_version(void);
const char* fpf_describe(void);

/* ---------------------------------------------------------------------------------------------------------------- LayerNorm
 * y[r, :] = (x[r, :] - mean) * rsqrt(var + eps) * gamma + beta, biased variance, fp32 statistics.
 * Replaces: common/opt_core/opt_core/kernels/ln/__init__.py:836 layer_norm (the standalone LN face; forms fp32 / bf16 /
 * bf16 out of ln/DESIGN.md:5-9 are the dtype_in / dtype_out pairs). */
typedef struct {
  int32_t abi_version;
  int32_t dtype_in;        /* FPF_DT_BF16 | FPF_DT_F32 */
  int32_t dtype_out;       /* FPF_DT_BF16 | FPF_DT_F32 */
  int32_t cols;            /* normalised width: bf16 input <= 1024, multiple of 8; fp32 input <= 512, multiple of 4 (8 for bf16 out) */
  int64_t rows;
  const void* x;
  int64_t x_row_stride;    /* elements between rows (>= cols) */
  void* y;
  int64_t y_row_stride;
  const float* gamma;      /* [cols] or NULL (= 1) */
  const float* beta;       /* [cols] or NULL (= 0) */
  float eps;
} FpfLnArgs;
int fpf_layernorm_fwd(const FpfLnArgs* a, void* stream, char* err, size_t errlen);

/* ---------------------------------------------------------------------------------------------------------------- transition
 * out = [x +] mask_r * W_o( silu(W_a n) * (W_b n) ),  n = LayerNorm(x) over c; hidden never leaves the chip.
 * Replaces: common/opt_core/opt_core/kernels/transition/__init__.py:1074 transition (row v2 semantics: mask and residual
 * folded, out may alias x) and common/opt_core/opt_core/attn/pair_fused.py:1519 transition. */
typedef struct {
  int32_t abi_version;
  int32_t dtype;           /* FPF_DT_BF16 (x, out, w_* bf16) | FPF_DT_F32 (all fp32) */
  int32_t c;               /* bf16: 128; fp32: any <= 384 */
  int32_t hidden;          /* bf16: multiple of 32; fp32: any */
  int64_t rows;
  const void* x;           /* [rows, c] contiguous */
  void* out;               /* [rows, c] contiguous; may equal x (each row is read before it is written) */
  const float* ln_w;       /* [c] or NULL */
  const float* ln_b;       /* [c] or NULL */
  float eps;
  const void* w_a;         /* [hidden, c] (silu branch) */
  const void* w_b;         /* [hidden, c] */
  const void* w_o;         /* [c, hidden] */
  const float* row_mask;   /* [rows] or NULL: the update is multiplied by it before the residual add */
  int32_t residual;        /* 1: out = x + update */
  const void* x_ln;        /* bf16 only: [rows, c] contiguous, the caller's own LayerNorm output of x, projected in place of LN(x)
                              (the exact-candidate construction, pair_fused.py:1089-1094 ln="stock"); the residual still adds x; NULL:
                              LN in the kernel */
  /* The single track's pair bias from the rows this call writes (bf16, c = 128; rows = B * pair_n * pair_n, a pair tensor
     [B, N, N, 128]): z_bias[b, h, i, j] = LN(out[b, i, j, :]) . w_z[h, :] (fp32 LayerNorm statistics, the normalised row
     rounded to bf16, fp32 accumulation) -- fpf_apb_bias_fwd's values on the written z, bitwise, without another pass over
     it.  The pass the reference runs separately on the resident z after the pair stack (the sequence pair bias of
     boltz2/opt/forward/pairfuse/bz_pairfuse.py:18-20, proj_z of boltz2/stock/src/boltz/model/layers/attentionv2.py:53-58)
     folded into the stack's last site.  w_z NULL: no bias. */
  const void* w_z;         /* [z_heads, 128] bf16 */
  const float* z_ln_w;     /* [128] or NULL (1) */
  const float* z_ln_b;     /* [128] or NULL (0) */
  float z_eps;
  int32_t z_heads;         /* 1 .. 32 */
  int64_t pair_n;          /* N */
  void* z_bias;            /* [B, z_heads, N, z_bias_ld] */
  int32_t z_bias_dtype;    /* FPF_DT_F32 | FPF_DT_BF16 */
  int64_t z_bias_ld;       /* >= N; <= 0 means N */
} FpfTransitionArgs;
int fpf_transition_fwd(const FpfTransitionArgs* a, void* stream, char* err, size_t errlen);

/* ---------------------------------------------------------------------------------------------------------------- triangle multiplication
 * x = LN_in(z); a = mask * sigmoid(x W_ag^T) * (x W_ap^T); b likewise;
 * X[i,j] = sum_k a[i,k] b[j,k] (outgoing) | sum_k a[k,i] b[k,j] (incoming);
 * update = sigmoid(x W_og^T) * (LN_out(X) W_o^T); out = [z +] update.
 * Replaces: common/opt_core/opt_core/kernels/trimul/__init__.py:1982 triangle_multiplication (op :3-11, the ten tensors of
 * WEIGHT_KEYS :171); the row `native` structure K1 -> batched contraction -> K3 (trimul/native/DESIGN.md:1-40).
 * Launches: K1 (LN_in + four gated projections + mask -> bf16 channel-major planes; the incoming variant writes them
 * transposed), the batched contraction over k, K3 (LN_out + W_o + output gate + residual). */
typedef struct {
  int32_t abi_version;
  int32_t dtype;           /* FPF_DT_BF16 (z, out, w_* bf16) | FPF_DT_F32 | FPF_DT_F32Z_BF16 (z, out fp32; w_* bf16; the LayerNorm
                              and the gate read z rounded to bf16, the residual adds the fp32 z; the whole op and the channels mode, no rows mode) */
  int32_t c_z;             /* bf16: 128 */
  int32_t c_h;             /* bf16: 128 */
  int64_t batch;
  int64_t n;
  const void* z;           /* [B, N, N, c_z] contiguous */
  void* out;               /* [B, N, N, c_z]; may equal z */
  const float* mask;       /* [B, N, N] (0 / 1) or NULL */
  const float* ln_in_w;    /* [c_z] */
  const float* ln_in_b;
  const float* ln_out_w;   /* [c_h] */
  const float* ln_out_b;
  const void* w_ag;        /* [c_h, c_z] */
  const void* w_ap;
  const void* w_bg;
  const void* w_bp;
  const void* w_o;         /* [c_z, c_h] */
  const void* w_og;        /* [c_z, c_z] */
  int32_t outgoing;        /* 1 outgoing, 0 incoming */
  int32_t residual;
  float eps;
  void* workspace;
  size_t workspace_bytes;
  /* The rows mode (bf16; common/opt_core/opt_core/mem/chunk.py:526 triangle_multiplication_chunked, mode "rows"): both
     operand planes are computed whole once from the input z (fpf_trimul_fixed_fwd into a caller buffer), then each call
     produces the output rows [row0, row0 + rows), holding only that row block's product plane
     (fpf_trimul_rows_workspace_bytes) instead of the whole one.  The operands never see an updated row, so out may be z
     (residual in place) in both directions, and every output element is the same arithmetic in the same order as in the
     whole op: the rows bitwise equal the whole op's.  rows = 0, row0 = 0, fixed_in = NULL: the whole op. */
  int64_t row0;
  int64_t rows;
  const void* fixed_in;    /* the A | B planes from fpf_trimul_fixed_fwd (same z, mask, weights, direction) */
} FpfTrimulArgs;
size_t fpf_trimul_workspace_bytes(int64_t batch, int64_t n, int32_t c_z, int32_t c_h, int32_t dtype);
int fpf_trimul_fwd(const FpfTrimulArgs* a, void* stream, char* err, size_t errlen);
/* The rows mode's operands: the A and B planes of the whole op (K1; bf16, fpf_trimul_fixed_bytes bytes, 16-byte aligned) into
   fixed_out; the workspace and row fields of `a` are not used.  No counterpart of its own in the reference (its rows mode
   builds the fixed operand inside the chunked driver, mem/chunk.py:526). */
size_t fpf_trimul_fixed_bytes(int64_t batch, int64_t n, int32_t c_h, int32_t dtype);
int fpf_trimul_fixed_fwd(const FpfTrimulArgs* a, void* fixed_out, void* stream, char* err, size_t errlen);
/* Workspace of a rows-mode call of `rows` rows: the product plane of the row block's cover by contraction tiles. */
size_t fpf_trimul_rows_workspace_bytes(int64_t batch, int64_t n, int64_t rows, int32_t c_h, int32_t dtype);
/* The channels mode (FPF_DT_BF16 or FPF_DT_F32Z_BF16, c_h = 128; common/opt_core/opt_core/mem/chunk.py:542-552,
   triangle_multiplication_chunked mode "channels"): the operand planes are built per block of `chunk` hidden channels (32, 64
   or 128: the largest not above chunk, 32 below that) and each block's products are written into the one full product
   plane, then the output stage runs over all rows.  The full plane is held because the output LayerNorm normalises over all
   hidden channels of a pixel.  The result equals fpf_trimul_fwd's bitwise; out may be z (residual).  The row fields of `a`
   must be 0 / NULL; the workspace (fpf_trimul_channels_workspace_bytes: the product plane + two planes of the block's
   channels) is a->workspace. */
size_t fpf_trimul_channels_workspace_bytes(int64_t batch, int64_t n, int64_t chunk, int32_t c_h, int32_t dtype);
int fpf_trimul_channels_fwd(const FpfTrimulArgs* a, int64_t chunk, void* stream, char* err, size_t errlen);

/* The same triangle multiplication without a caller workspace.  No counterpart in the reference: for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  The workspace
 * is a static per-device array of FPF_TRIMUL_NOALLOC_SCRATCH_BYTES (48 MiB, held by every GPU the library runs on until the
 * process ends): a call needing more (fpf_trimul_workspace_bytes; bf16 at B = 1: N <= 256) is refused with FPF_E_WORKSPACE.
 * a->workspace must be NULL and a->workspace_bytes 0.  The entry allocates nothing and uses the current device's array (the
 * device of `stream` must be current).  Calls that overlap on one GPU (two streams or host threads) share the array and race. */
#define FPF_TRIMUL_NOALLOC_SCRATCH_BYTES 50331648
int fpf_trimul_fwd_noalloc(const FpfTrimulArgs* a, void* stream, char* err, size_t errlen);

/* ---------------------------------------------------------------------------------------------------------------- triangle attention (op)
 * out[b,n,h,i,:] = softmax_j(scale q.k + bias[b,h,i,j], -inf where mask[b,n,j] == 0) @ v[b,n,h,j,:];
 * a row whose keys are all masked is the uniform mean of v over all keys.
 * Replaces: common/opt_core/opt_core/kernels/triattn/__init__.py:1094 triangle_attention (op :3-8); the reference's plain-C
 * call struct model is kernels/triattn_xla/csrc/triattn_cuda_abi.h:13-40. */
typedef struct {
  int32_t abi_version;
  int32_t dtype;           /* q / k / v / out: FPF_DT_BF16 (head_dim 32) | FPF_DT_F32 (head_dim <= 64) */
  int64_t B, N, H, S, D;
  const void* q;
  const void* k;
  const void* v;
  int64_t q_stride[5];     /* [B, N, H, S, D] element strides; stride[4] must be 1 */
  int64_t k_stride[5];
  int64_t v_stride[5];     /* v_layout 0 / 3: strides of [B, N, H, S, D]; v_layout 1 / 2: strides of [B, N, H, D, S] (V stored
                              transposed) */
  int32_t v_layout;        /* 0 | 1 | 2 | 3 (1, 2, 3 bf16 only); the last stride must be 1.  2 is the fused block's internal layout:
                              V^T with the keys of every 16-key block stored in the order 0-3, 8-11, 4-7, 12-15, q already
                              multiplied by scale * log2(e) (scale must be 1), fp32 bias times log2(e) (logits in log2 units) in
                              blocks (see bias), S a multiple of 64 up to 8192, out rows of 32 contiguous 16-byte aligned bf16.
                              3 is the same core with V as plain key rows [B, N, H, S, D] (keys in order) */
  const void* bias;        /* [B, H, S, S] (the [B,1,H,S,S] operand without its unit axis).  v_layout 2 / 3: each (b, h) plane is
                              S x S contiguous (bias_stride[2] = S, [3] = 1, 16-byte aligned) and holds 32 x 32 blocks (query
                              block qb, key block kb) at element 1024 (qb S / 32 + kb), each block as 4 pieces (keys 8j .. 8j + 7)
                              of 64 lanes (lane n + 32 g: query n, keys 8j + 4g .. 8j + 4g + 3) of 4 values */
  int32_t bias_dtype;      /* FPF_DT_F32 | FPF_DT_BF16 */
  int64_t bias_stride[4];  /* stride[3] must be 1 */
  const void* mask;        /* [B, N, S] or NULL, nonzero = attend */
  int32_t mask_dtype;      /* FPF_DT_U8 | FPF_DT_F32 */
  int64_t mask_stride[3];
  void* out;
  int64_t out_stride[5];   /* stride[4] must be 1 */
  float scale;
  const uint64_t* keep;    /* v_layout 2 / 3 only: the mask as a keep-bit table [B, N, S / 64 + 1] (per attention row: word 0 = flags,
                              bit 0 some key kept, bit 1 every key kept; word 1 + t = keep bits of keys 64 t .. 64 t + 63, all set
                              for a row with no kept key), or NULL with mask NULL (every key kept).  The fused block builds it from
                              its pair mask in its workspace; v_layout 2 / 3 with a mask and no table is refused (FPF_E_ARGS).  Other
                              layouts read `mask` and ignore this field. */
  void* workspace;         /* v_layout 2 / 3: device memory of fpf_triattn_workspace_bytes(B, N, H, S, v_layout) bytes (per work item
                              a flag the fast kernel writes and its fallback reads).  v_layout 0 / 1: NULL, or
                              fpf_triattn_stage_bytes(B, N, H, S, D, dtype) bytes or more, which runs a bf16 call with head_dim 32
                              on the block-layout core (the bias and the mask restaged there, v_layout 1's V^T too; q, k and
                              v_layout 0's v read in place; q / k / v rows and out rows of 32 contiguous 16-byte aligned bf16,
                              out_stride[3] = 32, q / k / v offsets within a (b, h) plane below 2^31 bytes); a call that does not
                              meet those conditions runs the op core as without */
  size_t workspace_bytes;
} FpfTriattnArgs;
int fpf_triattn_fwd(const FpfTriattnArgs* a, void* stream, char* err, size_t errlen);
/* Workspace of fpf_triattn_fwd for this layout (0 for v_layout 0 / 1; v_layout 2 and 3 take the same). */
size_t fpf_triattn_workspace_bytes(int64_t B, int64_t N, int64_t H, int64_t S, int32_t v_layout);
/* Staging workspace that puts a v_layout 0 / 1 call on the block-layout core: bf16, head_dim 32, S a multiple of 64 or at least
 * 128, up to 8192; 0 when the call's class has no staged route.  No counterpart in the reference (its op face routes S ranges
 * to tuned members, kernels/triattn/triattn_native/DESIGN.md:27-40; here the route is this workspace). */
size_t fpf_triattn_stage_bytes(int64_t B, int64_t N, int64_t H, int64_t S, int64_t D, int32_t dtype);

/* ---------------------------------------------------------------------------------------------------------------- triangle attention (block)
 * The fused block: prologue (LN -> q|k|v|g and the pair-bias projection, reading z or z^T by address) -> core -> epilogue
 * (sigmoid(g) * o @ W_o^T, written as an update in z's frame or added to z in place, transposed scatter for the ending node).
 * Replaces: common/opt_core/opt_core/attn/pair_fused.py:1500 tri_attn_block (prologue :1136, core_attention :1391,
 * epilogue :1416; weights as pack_triattn_weights :679 packs them: w_qkvg [4HD, C] rows q|k|v|g, w_b [H, C], w_o [C, HD]). */
typedef struct {
  int32_t abi_version;
  int32_t dtype;           /* FPF_DT_BF16 (C = 128, H*D = 128, D = 32) | FPF_DT_F32 */
  int64_t B, N;
  int32_t C, H, D;
  const void* z;           /* [B, N, N, C] contiguous, z's own frame */
  const void* mask;        /* [B, N, N] pair mask in z's frame or NULL, nonzero = keep */
  int32_t mask_dtype;      /* FPF_DT_U8 | FPF_DT_F32 */
  const float* ln_w;       /* [C] or NULL */
  const float* ln_b;
  float eps;
  const void* w_qkvg;      /* [4*H*D, C] */
  const void* w_b;         /* [H, C] */
  const void* w_o;         /* [C, H*D] */
  int32_t ending;          /* 0 starting node, 1 ending node (attention over z^T) */
  int32_t residual;        /* 1: z += update in place (z must then be writable: out == z) */
  void* out;               /* residual: == z; else the update [B, N, N, C] in z's frame */
  float scale;             /* <= 0: 1/sqrt(D) */
  void* workspace;
  size_t workspace_bytes;
  int64_t row0;            /* attention rows [row0, row0 + rows) only (bf16; the `big` row-chunked driver); rows <= 0: all N */
  int64_t rows;
  const float* bias_in;    /* NULL: the block computes the bias; else the full bias of fpf_triattn_bias_fwd (fpf_triattn_bias_bytes
                              bytes; required with a row range: every attention row needs the bias of every pair) */
  int32_t mask_frame;      /* 0: mask in z's frame (the ending node reads its columns); 1: mask already in the attention
                              frame (for the ending node the transposed pair mask, so every key row is contiguous); other values:
                              FPF_E_ARGS */
  const float* b_g;        /* [H*D] gate projection bias (g = x_ln W_g^T + b_g, before the sigmoid) or NULL; pair_fused.py:731-736 */
  const float* b_o;        /* [C] output projection bias (u = (sigmoid(g) o) W_o^T + b_o) or NULL; pair_fused.py:738 */
  const void* x_ln;        /* bf16 whole block only: [B, N, N, C] contiguous, the caller's LayerNorm output in the attention frame
                              (LN(z), or LN(z^T) for the ending node), projected in place of the in-kernel LayerNorm for q, k, v, the
                              bias and the gate (pair_fused.py:1019-1029, :1151-1160 ln="stock"); the residual still updates z */
} FpfTriattnBlockArgs;
/* Workspace for `rows` attention rows (rows <= 0: all N). */
size_t fpf_triattn_block_workspace_bytes(int64_t B, int64_t N, int64_t rows, int32_t C, int32_t H, int32_t D, int32_t dtype);
int fpf_triattn_block_fwd(const FpfTriattnBlockArgs* a, void* stream, char* err, size_t errlen);

/* The bias pass of the row-chunked (`big`) triangle-attention block: bias[b, h, i, j] = LN(x)[i, j] . w_b[h] for every pixel of
 * the attention frame (x = z or z^T), fp32, bf16 block only.  Replaces pass 1 of common/opt_core/opt_core/mem/chunk.py:424
 * (triangle_attention_chunked: the full bias assembled block by block before the per-row attention pass). */
typedef struct {
  int32_t abi_version;
  int32_t dtype;           /* FPF_DT_BF16 */
  int64_t B, N;
  int32_t C, H, D;
  const void* z;           /* [B, N, N, C] */
  const float* ln_w;
  const float* ln_b;
  float eps;
  const void* w_qkvg;      /* may be NULL (not read) */
  const void* w_b;         /* [H, C] */
  int32_t ending;
  float* bias;             /* fp32 out, fpf_triattn_bias_bytes(B, N, H, dtype) bytes, in the units and layout fpf_triattn_block_fwd's
                              core takes: for the bf16 block up to N = 8192 (the v_layout 2 core) [B, H, Np, Np] with Np = N
                              rounded up to 64, times log2(e), in the 32 x 32 register-order blocks (the padding rows and
                              columns are not written); else [B, H, N, N] as is, row-major */
} FpfTriattnBiasArgs;
int fpf_triattn_bias_fwd(const FpfTriattnBiasArgs* a, void* stream, char* err, size_t errlen);
/* Bytes of fpf_triattn_bias_fwd's output (no counterpart in the reference: its bias is a torch tensor the driver allocates). */
size_t fpf_triattn_bias_bytes(int64_t B, int64_t N, int32_t H, int32_t dtype);

/* ---------------------------------------------------------------------------------------------------------------- triangle attention (block stages)
 * The block's prologue and epilogue as separate calls, for callers that run their own core between them.
 * Prologue replaces common/opt_core/opt_core/attn/pair_fused.py:1136 prologue (-> q, k, v, g, bias in the attention frame
 * x = z or z^T): x_ln = LN(x); q|k|v|g = x_ln W_qkvg^T; bias = x_ln W_b^T.
 * Epilogue replaces pair_fused.py:1416 epilogue: u = (sigmoid(g) * o) W_o^T, written in z's frame (the ending node's u[i, j]
 * lands at pixel (j, i)), or added to z in place. */
typedef struct {
  int32_t abi_version;
  int32_t dtype;           /* FPF_DT_BF16 (C = 128, H*D = 128, D = 32) | FPF_DT_F32 (C, H*D <= 128) */
  int64_t B, N;
  int32_t C, H, D;
  const void* z;           /* [B, N, N, C] contiguous, z's own frame */
  const float* ln_w;       /* [C] or NULL */
  const float* ln_b;
  float eps;
  const void* w_qkvg;      /* [4*H*D, C] rows q | k | v | g */
  const void* w_b;         /* [H, C] */
  int32_t ending;          /* 1: attention frame x = z^T (read by address) */
  void* q;                 /* [B, I, H, J, D] contiguous */
  void* k;                 /* [B, I, H, J, D] */
  void* v;                 /* bf16: [B, I, H, D, v_ld] (stored transposed, the core's v_layout 1; columns >= N are padding);
                              fp32: [B, I, H, J, D] */
  int64_t v_ld;            /* bf16: elements between V^T rows, >= N rounded up to 32 and a multiple of 8; fp32: ignored */
  void* g;                 /* [B, I, J, H*D] pre-sigmoid */
  float* bias;             /* [B, H, I, J] fp32 (the [B,1,H,I,J] operand without its unit axis) */
  const float* b_g;        /* [H*D] gate projection bias added to g, or NULL */
  const void* x_ln;        /* bf16 only: [B, N, N, C] contiguous, the caller's LayerNorm output in the attention frame, projected in
                              place of the in-kernel LayerNorm (ln="stock"); NULL: LN in the kernel */
} FpfTriattnPrologueArgs;
int fpf_triattn_prologue_fwd(const FpfTriattnPrologueArgs* a, void* stream, char* err, size_t errlen);

typedef struct {
  int32_t abi_version;
  int32_t dtype;           /* as the prologue */
  int64_t B, N;
  int32_t C, H, D;
  const void* o;           /* [B, I, H, J, D] contiguous (the core's output) */
  const void* g;           /* [B, I, J, H*D] pre-sigmoid */
  const void* w_o;         /* [C, H*D] */
  int32_t ending;
  int32_t residual;        /* 1: out is z and z += u in place */
  void* out;               /* [B, N, N, C] in z's frame */
  const float* b_o;        /* [C] output projection bias added to u, or NULL */
} FpfTriattnEpilogueArgs;
int fpf_triattn_epilogue_fwd(const FpfTriattnEpilogueArgs* a, void* stream, char* err, size_t errlen);

/* ---------------------------------------------------------------------------------------------------------------- attention with a pair bias
 * The single track's attention (and a sample batch's token attention sharing one bias):
 * out[s,n,h,:] = sigmoid(gate[s,n,h,:]) * softmax_m(scale q[s,n,h,:].k[s,m,h,:] + bias[s|0,h,n,m], keys with key_mask[s|0,m] == 0
 *                excluded) @ v[s,m,h,:]; a sample whose keys are all masked gives the uniform mean of v over all keys.
 * fp32 arithmetic for fp32 or bf16 storage.
 * Replaces: common/opt_core/opt_core/attn/apb_core.py:89 pair_bias_attention (its "rows" and "shnd" layouts are strided views
 * of [S, N, H, D] here); the stock statement is boltz2/stock/src/boltz/model/layers/attentionv2.py:98-111. */
typedef struct {
  int32_t abi_version;
  int32_t dtype;           /* q / k / v / gate / out: FPF_DT_F32 | FPF_DT_BF16 */
  int64_t S, N, NK, H, D;  /* samples, queries, keys, heads, head_dim (16 | 24 | 32 | 48 | 64) */
  const void* q;           /* [S, N, H, D] element strides below, stride[3] = 1 */
  const void* k;           /* [S, NK, H, D] */
  const void* v;           /* [S, NK, H, D] */
  int64_t q_stride[4];
  int64_t k_stride[4];
  int64_t v_stride[4];
  const void* gate;        /* [S, N, H, D] pre-sigmoid, or NULL (no gate) */
  int64_t gate_stride[4];
  const void* bias;        /* [SB, H, N, NK]: stride[0] = 0 shares one plane across the samples */
  int32_t bias_dtype;      /* FPF_DT_F32 | FPF_DT_BF16 */
  int64_t bias_stride[4];  /* stride[3] = 1 */
  const void* key_mask;    /* [S | 1, NK] nonzero = attend, or NULL */
  int32_t mask_dtype;      /* FPF_DT_U8 | FPF_DT_F32 */
  int64_t mask_stride[2];  /* stride[0] = 0 shares one mask across the samples */
  void* out;               /* [S, N, H, D] */
  int64_t out_stride[4];
  float scale;             /* > 0 (the face passes head_dim ** -0.5 by default) */
} FpfApbArgs;
int fpf_apb_fwd(const FpfApbArgs* a, void* stream, char* err, size_t errlen);

/* The pair-bias producer: bias[b, h, i, j] = LN(z[b, i, j, :]) . w_z[h, :] over every pixel (fp32 LayerNorm statistics, the
 * normalised row rounded to bf16, fp32 accumulation), head-major with a row pitch, fp32 or bf16.
 * Replaces: the `producer` boundary of common/opt_core/opt_core/kernels/apb (DESIGN.md:5-7); the stock statement is the
 * proj_z of boltz2/stock/src/boltz/model/layers/attentionv2.py:53-58 (LayerNorm(c_z) -> Linear(c_z, H, bias=False) -> heads first). */
typedef struct {
  int32_t abi_version;
  int32_t dtype;           /* z: FPF_DT_BF16 */
  int64_t B, N;
  int32_t C, H;            /* C = 128, 1 <= H <= 32 */
  const void* z;           /* [B, N, N, C] contiguous */
  const float* ln_w;       /* [C] or NULL (1) */
  const float* ln_b;       /* [C] or NULL (0) */
  float eps;
  const void* w_z;         /* [H, C] bf16 */
  void* bias;              /* [B, H, N, bias_ld] out */
  int32_t bias_dtype;      /* FPF_DT_F32 | FPF_DT_BF16 */
  int64_t bias_ld;         /* >= N; <= 0 means N */
} FpfApbBiasArgs;
int fpf_apb_bias_fwd(const FpfApbBiasArgs* a, void* stream, char* err, size_t errlen);

#ifdef __cplusplus
}
#endif
#endif /* FPF_HIP_H */
