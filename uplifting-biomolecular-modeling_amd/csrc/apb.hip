// Attention with a pair bias: the Pairformer single track's AttentionPairBias core, and the token attention of a sample batch
// sharing one bias (S samples, one [H, N, NK] bias plane, or one plane per sample).  Replaces
// common/opt_core/opt_core/attn/apb_core.py:89 (pair_bias_attention; the stock statement is
// boltz2/stock/src/boltz/model/layers/attentionv2.py:98-111, which runs in fp32 with autocast off).
//
// fp32 arithmetic throughout, for fp32 or bf16 storage: the single track's work is small next to the pair track (at
// N = 512, 16 heads x 24: 0.4 GFLOP per block against ~500 for the pair sites), so the kernel spends its effort on exact
// statistics (fp32 logits; exponentials by v_exp_f32 on logits kept in log2 units, q and the bias carrying log2(e)) rather
// than on the matrix cores.  A workgroup = 64 queries (one per lane) of one (sample, head) and W waves (8 for head dims up
// to 24, else 4: the register budget); wave w walks its share of the keys in 32-key tiles staged in a private LDS slot (K, V, the
// 64 x 32 bias tile and the keep flags), with an online softmax per 8-key chunk (chunk max, one rescale, exp per key); the
// W partial states are combined through LDS and the sigmoid gate applied on the way out.  A sample whose keys are all masked
// attends uniformly to every key (logits 0), the convention of the reference faces.
#include <algorithm>
#include <type_traits>

#include "fpf_common.h"

namespace fpf {

constexpr int AP_Q = 64;     // queries per workgroup
constexpr int AP_KT = 32;    // keys per staged tile
constexpr float AP_LOG2E = 1.4426950408889634f;
template <int D>
constexpr int ap_waves() { return D <= 24 ? 8 : 4; }   // waves per workgroup: the key range is split W ways

struct ApbParams {
  const void* q;
  const void* k;
  const void* v;
  const void* gate;
  const void* bias;
  const void* mask;
  void* out;
  int64_t qs[4], ks[4], vs[4], gs[4], bs[4], os[4], ms[2];
  int64_t S, N, NK, H;
  float scale;
  int bias_bf16, mask_f32;
  int vec;                       // fp32 K / V / bias in 16-byte aligned rows (NK a multiple of 4): the tiles load 16 bytes a lane
};

__device__ __forceinline__ float ldv(const float* p, int64_t o) { return p[o]; }
__device__ __forceinline__ float ldv(const uint16_t* p, int64_t o) { return bf2f(p[o]); }
__device__ __forceinline__ void stv(float* p, int64_t o, float x) { p[o] = x; }
__device__ __forceinline__ void stv(uint16_t* p, int64_t o, float x) { p[o] = f2bf(x); }

__device__ __forceinline__ bool apb_keep(const ApbParams& p, int64_t s, int64_t j) {
  if (!p.mask) return true;
  const int64_t o = s * p.ms[0] + j * p.ms[1];
  return p.mask_f32 ? static_cast<const float*>(p.mask)[o] != 0.0f : static_cast<const uint8_t*>(p.mask)[o] != 0;
}

// Orders a wave's own LDS writes before its reads of other lanes' data (a wave's LDS operations execute in order).
__device__ __forceinline__ void apb_wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <typename T, int D, int AP_W, bool VEC>
__global__ void __launch_bounds__(64 * AP_W) apb_fwd_kernel(const ApbParams p) {
  // per-wave slots: K and V [AP_KT][D] (16-byte rows, read as broadcasts), bias [AP_Q][AP_KT + 1], keep [AP_KT]; reused
  // after the key loop for the partial states [AP_W][AP_Q][D + 2] (o, m, l) of the combine
  static_assert(D % 4 == 0, "K / V rows are read 16 bytes at a time");
  constexpr int KV = AP_KT * D, BT = AP_Q * (AP_KT + 1), SLOT = 2 * KV + BT + AP_KT;
  constexpr int PART = AP_W * AP_Q * (D + 2);
  __shared__ __attribute__((aligned(16))) float smem[(AP_W * SLOT > PART) ? AP_W * SLOT : PART];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63;
  const int64_t nqt = cdiv(p.N, AP_Q);
  const int64_t w = blockIdx.x;
  const int64_t qt = w % nqt, sh = w / nqt, h = sh % p.H, s = sh / p.H;
  const int64_t i = qt * AP_Q + l;
  const bool qlive = i < p.N;
  const T* qp = static_cast<const T*>(p.q);
  const T* kp = static_cast<const T*>(p.k);
  const T* vp = static_cast<const T*>(p.v);

  // a sample with no kept key attends uniformly to every key
  bool any = false;
  for (int64_t j = tid; j < p.NK && !any; j += 64 * AP_W) any = apb_keep(p, s, j);
  const bool dead = !__syncthreads_or(any);

  float qv[D], ov[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    qv[d] = qlive ? ldv(qp, s * p.qs[0] + i * p.qs[1] + h * p.qs[2] + d) * (p.scale * AP_LOG2E) : 0.f;
    ov[d] = 0.f;
  }
  float m = -INFINITY, lsum = 0.f;

  float* sK = smem + wave * SLOT;
  float* sV = sK + KV;
  float* sB = sV + KV;
  float* sKeep = sB + BT;
  const int64_t ntile = cdiv(p.NK, AP_KT), per = cdiv(ntile, AP_W);
  const int64_t t0 = wave * per, t1 = std::min<int64_t>(ntile, t0 + per);
  const int64_t bplane = s * p.bs[0] + h * p.bs[1];       // bs[0] = 0: one plane shared by the samples
  // a tile's K / V values (NKV per lane each), then its bias values (NB per lane): each group's loads are all issued before
  // its first LDS store, so the tile waits for two memory latencies rather than one per element
  constexpr int NKV = AP_KT * D / 64, NB = AP_Q * AP_KT / 64;
  static_assert(AP_KT * D % 64 == 0 && AP_Q * AP_KT % 64 == 0, "whole rounds of 64 lanes");
  for (int64_t t = t0; t < t1; ++t) {
    const int64_t k0 = t * AP_KT;
    if constexpr (VEC) {
      // K / V: key row kk as D / 4 16-byte pieces, D / 8 per lane; bias: 64 query rows x 8 pieces, 8 per lane
      constexpr int NV4 = AP_KT * D / 4 / 64, NB4 = AP_Q * AP_KT / 4 / 64;
      static_assert(AP_KT * D / 4 % 64 == 0, "whole rounds of 64 lanes");
      const float* kf = reinterpret_cast<const float*>(kp);
      const float* vf = reinterpret_cast<const float*>(vp);
      const float* bf = static_cast<const float*>(p.bias);
      f32x4 rk[NV4], rv[NV4], rb[NB4];
#pragma unroll
      for (int r = 0; r < NV4; ++r) {
        const int e = l + 64 * r, kk = e / (D / 4), c4 = e - kk * (D / 4);
        const int64_t j = k0 + kk;
        const bool ok = j < p.NK;
        rk[r] = ok ? *reinterpret_cast<const f32x4*>(kf + s * p.ks[0] + j * p.ks[1] + h * p.ks[2] + 4 * c4) : f32x4{0.f, 0.f, 0.f, 0.f};
        rv[r] = ok ? *reinterpret_cast<const f32x4*>(vf + s * p.vs[0] + j * p.vs[1] + h * p.vs[2] + 4 * c4) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int r = 0; r < NB4; ++r) {
        const int e = l + 64 * r, qq = e / (AP_KT / 4), c = e - qq * (AP_KT / 4);
        const int64_t ii = qt * AP_Q + qq, j = k0 + 4 * c;
        rb[r] = ii < p.N && j < p.NK ? *reinterpret_cast<const f32x4*>(bf + bplane + ii * p.bs[2] + j) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int r = 0; r < NV4; ++r) {
        *reinterpret_cast<f32x4*>(sK + 4 * (l + 64 * r)) = rk[r];
        *reinterpret_cast<f32x4*>(sV + 4 * (l + 64 * r)) = rv[r];
      }
#pragma unroll
      for (int r = 0; r < NB4; ++r) {
        const int e = l + 64 * r, qq = e / (AP_KT / 4), c = e - qq * (AP_KT / 4);
#pragma unroll
        for (int u = 0; u < 4; ++u) sB[qq * (AP_KT + 1) + 4 * c + u] = rb[r][u] * AP_LOG2E;
      }
    } else {
    {
      float rk[NKV], rv[NKV];
#pragma unroll
      for (int r = 0; r < NKV; ++r) {
        const int e = l + 64 * r, kk = e / D, d = e - kk * D;
        const int64_t j = k0 + kk;
        const bool ok = j < p.NK;
        rk[r] = ok ? ldv(kp, s * p.ks[0] + j * p.ks[1] + h * p.ks[2] + d) : 0.f;
        rv[r] = ok ? ldv(vp, s * p.vs[0] + j * p.vs[1] + h * p.vs[2] + d) : 0.f;
      }
#pragma unroll
      for (int r = 0; r < NKV; ++r) {
        sK[l + 64 * r] = rk[r];
        sV[l + 64 * r] = rv[r];
      }
    }
    {
      float rb[NB];
#pragma unroll
      for (int r = 0; r < NB; ++r) {
        const int e = l + 64 * r, qq = e / AP_KT, kk = e - qq * AP_KT;
        const int64_t ii = qt * AP_Q + qq, j = k0 + kk;
        float bv = 0.f;
        if (ii < p.N && j < p.NK) {
          const int64_t o = bplane + ii * p.bs[2] + j;
          bv = p.bias_bf16 ? bf2f(static_cast<const uint16_t*>(p.bias)[o]) : static_cast<const float*>(p.bias)[o];
        }
        rb[r] = bv;
      }
#pragma unroll
      for (int r = 0; r < NB; ++r) {
        const int e = l + 64 * r, qq = e / AP_KT, kk = e - qq * AP_KT;
        sB[qq * (AP_KT + 1) + kk] = rb[r] * AP_LOG2E;
      }
    }
    }
    if (l < AP_KT) sKeep[l] = (k0 + l < p.NK && (dead || apb_keep(p, s, k0 + l))) ? 1.f : 0.f;
    apb_wave_sync();
    // 8 keys at a time: logits, one rescale per chunk (the keep flags are per key, so a chunk is dead for every lane or for
    // none), exp and P.V; K / V rows are the same for every lane (broadcast 16-byte reads)
#pragma unroll 1
    for (int c8 = 0; c8 < AP_KT; c8 += 8) {
      float lg[8];
      float cmax = -INFINITY;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int kk = c8 + u;
        const f32x4* kr = reinterpret_cast<const f32x4*>(sK + kk * D);
        float a = sB[l * (AP_KT + 1) + kk];
#pragma unroll
        for (int d4 = 0; d4 < D / 4; ++d4) {
          const f32x4 kv = kr[d4];
#pragma unroll
          for (int e = 0; e < 4; ++e) a = fmaf(qv[4 * d4 + e], kv[e], a);
        }
        if (dead) a = 0.f;
        lg[u] = sKeep[kk] != 0.f ? a : -INFINITY;
        cmax = fmaxf(cmax, lg[u]);
      }
      if (cmax == -INFINITY) continue;
      const float mn = fmaxf(m, cmax);
      const float alpha = fast_exp2(m - mn);            // m = -inf before the first live chunk: alpha = 0 on zeros
      lsum *= alpha;
#pragma unroll
      for (int d = 0; d < D; ++d) ov[d] *= alpha;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float pe = fast_exp2(lg[u] - mn);
        lsum += pe;
        const f32x4* vr = reinterpret_cast<const f32x4*>(sV + (c8 + u) * D);
#pragma unroll
        for (int d4 = 0; d4 < D / 4; ++d4) {
          const f32x4 vv = vr[d4];
#pragma unroll
          for (int e = 0; e < 4; ++e) ov[4 * d4 + e] = fmaf(pe, vv[e], ov[4 * d4 + e]);
        }
      }
      m = mn;
    }
    apb_wave_sync();                                     // the slot is rewritten by the next tile
  }

  // combine the W key ranges
  __syncthreads();
  float* part = smem + (wave * AP_Q + l) * (D + 2);
#pragma unroll
  for (int d = 0; d < D; ++d) part[d] = ov[d];
  part[D] = m;
  part[D + 1] = lsum;
  __syncthreads();
  if (wave != 0 || !qlive) return;
  float M = -INFINITY;
#pragma unroll
  for (int ww = 0; ww < AP_W; ++ww) M = fmaxf(M, smem[(ww * AP_Q + l) * (D + 2) + D]);
  float L = 0.f;
  float o[D];
#pragma unroll
  for (int d = 0; d < D; ++d) o[d] = 0.f;
#pragma unroll
  for (int ww = 0; ww < AP_W; ++ww) {
    const float* pw = smem + (ww * AP_Q + l) * (D + 2);
    const float f = pw[D] == -INFINITY ? 0.f : fast_exp2(pw[D] - M);
    L += f * pw[D + 1];
#pragma unroll
    for (int d = 0; d < D; ++d) o[d] = fmaf(f, pw[d], o[d]);
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  const T* gp = static_cast<const T*>(p.gate);
  T* op = static_cast<T*>(p.out);
#pragma unroll
  for (int d = 0; d < D; ++d) {
    float y = o[d] * inv;
    if (gp) y *= 1.0f / (1.0f + expf(-ldv(gp, s * p.gs[0] + i * p.gs[1] + h * p.gs[2] + d)));
    stv(op, s * p.os[0] + i * p.os[1] + h * p.os[2] + d, y);
  }
}

template <typename T, int DD>
static void apb_launch_dd(const ApbParams& p, int64_t blocks, hipStream_t st) {
  if constexpr (std::is_same<T, float>::value) {
    if (p.vec) {
      hipLaunchKernelGGL((apb_fwd_kernel<T, DD, ap_waves<DD>(), true>), dim3((unsigned)blocks), dim3(64 * ap_waves<DD>()), 0, st, p);
      return;
    }
  }
  hipLaunchKernelGGL((apb_fwd_kernel<T, DD, ap_waves<DD>(), false>), dim3((unsigned)blocks), dim3(64 * ap_waves<DD>()), 0, st, p);
}

template <typename T>
static int apb_launch_d(const ApbParams& p, int64_t D, hipStream_t st, char* err, size_t errlen) {
  const int64_t blocks = p.S * p.H * cdiv(p.N, AP_Q);
  if (blocks > 0x7fffffffLL) return fail(err, errlen, FPF_E_SHAPE, "grid too large");
#define FPF_APB(DD)                                                                                   \
  if (D == DD) {                                                                                      \
    apb_launch_dd<T, DD>(p, blocks, st);                                                              \
    return launched(err, errlen, "apb_fwd_kernel");                                                   \
  }
  FPF_APB(16) FPF_APB(24) FPF_APB(32) FPF_APB(48) FPF_APB(64)
#undef FPF_APB
  return fail(err, errlen, FPF_E_SHAPE, "head_dim %lld (served: 16, 24, 32, 48, 64)", (long long)D);
}

}  // namespace fpf

extern "C" int fpf_apb_fwd(const FpfApbArgs* a, void* stream, char* err, size_t errlen) {
  using namespace fpf;
  FPF_CHECK_VERSION(a);
  if (!a->q || !a->k || !a->v || !a->bias || !a->out) return fail(err, errlen, FPF_E_ARGS, "q / k / v / bias / out is NULL");
  if (a->S < 0 || a->N < 0 || a->NK < 0 || a->H <= 0 || a->D <= 0) return fail(err, errlen, FPF_E_SHAPE, "negative extent");
  if (a->S == 0 || a->N == 0) return FPF_OK;
  if (a->NK == 0) return fail(err, errlen, FPF_E_SHAPE, "no keys (NK = 0)");
  if (!(a->dtype == FPF_DT_F32 || a->dtype == FPF_DT_BF16)) return fail(err, errlen, FPF_E_DTYPE, "dtype %d", a->dtype);
  if (!(a->bias_dtype == FPF_DT_F32 || a->bias_dtype == FPF_DT_BF16)) return fail(err, errlen, FPF_E_DTYPE, "bias_dtype %d", a->bias_dtype);
  if (a->key_mask && !(a->mask_dtype == FPF_DT_U8 || a->mask_dtype == FPF_DT_F32)) return fail(err, errlen, FPF_E_DTYPE, "mask_dtype %d", a->mask_dtype);
  if (a->q_stride[3] != 1 || a->k_stride[3] != 1 || a->v_stride[3] != 1 || a->out_stride[3] != 1 || a->bias_stride[3] != 1 ||
      (a->gate && a->gate_stride[3] != 1))
    return fail(err, errlen, FPF_E_SHAPE, "the innermost (head_dim / key) strides must be 1");
  if (!(a->scale > 0.f) || !(a->scale < INFINITY)) return fail(err, errlen, FPF_E_ARGS, "scale must be finite and > 0");
  ApbParams p{};
  p.q = a->q;
  p.k = a->k;
  p.v = a->v;
  p.gate = a->gate;
  p.bias = a->bias;
  p.mask = a->key_mask;
  p.out = a->out;
  for (int t = 0; t < 4; ++t) {
    p.qs[t] = a->q_stride[t];
    p.ks[t] = a->k_stride[t];
    p.vs[t] = a->v_stride[t];
    p.gs[t] = a->gate_stride[t];
    p.bs[t] = a->bias_stride[t];
    p.os[t] = a->out_stride[t];
  }
  p.ms[0] = a->mask_stride[0];
  p.ms[1] = a->mask_stride[1];
  p.S = a->S;
  p.N = a->N;
  p.NK = a->NK;
  p.H = a->H;
  p.scale = a->scale;
  p.bias_bf16 = a->bias_dtype == FPF_DT_BF16;
  p.mask_f32 = a->mask_dtype == FPF_DT_F32;
  const auto a16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  p.vec = a->dtype == FPF_DT_F32 && !p.bias_bf16 && a->NK % 4 == 0 && a16(a->k) && a16(a->v) && a16(a->bias) &&
          ((p.ks[0] | p.ks[1] | p.ks[2] | p.vs[0] | p.vs[1] | p.vs[2] | p.bs[0] | p.bs[1] | p.bs[2]) & 3) == 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return a->dtype == FPF_DT_F32 ? apb_launch_d<float>(p, a->D, st, err, errlen) : apb_launch_d<uint16_t>(p, a->D, st, err, errlen);
}
