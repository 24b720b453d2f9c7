// Standalone LayerNorm (HBM-bound): 16 lanes per row, 128-bit loads and stores, fp32 statistics with an exact two-pass
// variance held in registers (one read of x, one write of y).  y is written with non-temporal stores: streamed out
// without displacing cached lines (bf16 at 589,824 x 128 on MI355X: 56 -> 50 us, a plain 16-byte copy of the same bytes
// 49-54 us).
// Replaces the reference's LN face common/opt_core/opt_core/kernels/ln/__init__.py:836 (layer_norm).
#include "fpf_common.h"

namespace fpf {

// 16 lanes per row, LN_RPT rows per thread: every row's loads are issued before any reduction so each lane keeps LN_RPT
// 16-byte requests in flight (a single row per thread leaves the kernel latency-bound, not bandwidth-bound).
constexpr int LN_RPT = 4;

template <typename TI, typename TO, int VPL>
__global__ void __launch_bounds__(256) ln_rows_kernel(const TI* __restrict__ x, int64_t xs, TO* __restrict__ y, int64_t ys,
                                                      const float* __restrict__ gamma, const float* __restrict__ beta,
                                                      int64_t rows, int cols, float eps) {
  constexpr int E = 16 / sizeof(TI);                 // elements per 16-byte vector
  const int lane = threadIdx.x & 15;
  const int64_t row0 = (int64_t)blockIdx.x * (16 * LN_RPT) + (threadIdx.x >> 4);
  float v[LN_RPT][VPL * E];
#pragma unroll
  for (int rr = 0; rr < LN_RPT; ++rr) {
    const int64_t row = row0 + 16 * rr;
#pragma unroll
    for (int c = 0; c < VPL; ++c) {
      const int e0 = (lane + 16 * c) * E;
      u32x4 raw = {0, 0, 0, 0};
      if (row < rows && e0 < cols) raw = *reinterpret_cast<const u32x4*>(x + row * xs + e0);
      if constexpr (sizeof(TI) == 4) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[rr][c * E + e] = __uint_as_float(raw[e]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[rr][c * E + 2 * e] = lo_bf(raw[e]);
          v[rr][c * E + 2 * e + 1] = hi_bf(raw[e]);
        }
      }
    }
  }
  float gw[VPL * E], bw[VPL * E];
#pragma unroll
  for (int c = 0; c < VPL; ++c) {
    const int e0 = (lane + 16 * c) * E;
#pragma unroll
    for (int e = 0; e < E; e += 4) {
      const bool ok = e0 + e < cols;
      const f32x4 g4 = (gamma && ok) ? *reinterpret_cast<const f32x4*>(gamma + e0 + e) : f32x4{1, 1, 1, 1};
      const f32x4 b4 = (beta && ok) ? *reinterpret_cast<const f32x4*>(beta + e0 + e) : f32x4{0, 0, 0, 0};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        gw[c * E + e + u] = g4[u];
        bw[c * E + e + u] = b4[u];
      }
    }
  }
#pragma unroll
  for (int rr = 0; rr < LN_RPT; ++rr) {
    const int64_t row = row0 + 16 * rr;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < VPL * E; ++i) s += v[rr][i];
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) s += __shfl_xor(s, o, 16);
    const float mean = s / (float)cols;
    float q = 0.f;
#pragma unroll
    for (int c = 0; c < VPL; ++c) {
      if ((lane + 16 * c) * E < cols) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const float d = v[rr][c * E + e] - mean;
          q += d * d;
        }
      }
    }
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) q += __shfl_xor(q, o, 16);
    const float rstd = 1.0f / sqrtf(q / (float)cols + eps);
    if (row >= rows) continue;
#pragma unroll
    for (int c = 0; c < VPL; ++c) {
      const int e0 = (lane + 16 * c) * E;
      if (e0 >= cols) continue;
      float o[E];
#pragma unroll
      for (int e = 0; e < E; ++e) o[e] = (v[rr][c * E + e] - mean) * rstd * gw[c * E + e] + bw[c * E + e];
      if constexpr (sizeof(TO) == 4) {
#pragma unroll
        for (int e = 0; e < E; e += 4)
          __builtin_nontemporal_store(f32x4{o[e], o[e + 1], o[e + 2], o[e + 3]}, reinterpret_cast<f32x4*>(y + row * ys + e0 + e));
      } else if constexpr (E == 8) {
        __builtin_nontemporal_store(u32x4{pack2(o[0], o[1]), pack2(o[2], o[3]), pack2(o[4], o[5]), pack2(o[6], o[7])},
                                    reinterpret_cast<u32x4*>(y + row * ys + e0));
      } else {
        __builtin_nontemporal_store(u32x2{pack2(o[0], o[1]), pack2(o[2], o[3])}, reinterpret_cast<u32x2*>(y + row * ys + e0));
      }
    }
  }
}

template <typename TI, typename TO>
static int launch_ln(const FpfLnArgs* a, hipStream_t st, char* err, size_t errlen) {
  constexpr int E = 16 / sizeof(TI);
  const int vpl_need = (int)cdiv(a->cols, 16 * E);
  const dim3 grid((unsigned)cdiv(a->rows, 16 * LN_RPT)), block(256);
  const TI* x = static_cast<const TI*>(a->x);
  TO* y = static_cast<TO*>(a->y);
#define FPF_LN(VPL)                                                                                                    \
  if (vpl_need <= VPL) {                                                                                              \
    hipLaunchKernelGGL((ln_rows_kernel<TI, TO, VPL>), grid, block, 0, st, x, a->x_row_stride, y, a->y_row_stride,     \
                       a->gamma, a->beta, a->rows, a->cols, a->eps);                                                  \
    return launched(err, errlen, "fpf_layernorm_fwd");                                                               \
  }
  FPF_LN(1) FPF_LN(2) FPF_LN(4) FPF_LN(8)
#undef FPF_LN
  return fail(err, errlen, FPF_E_SHAPE, "cols=%d above %d", a->cols, E == 8 ? 1024 : 512);
}

}  // namespace fpf

extern "C" int fpf_abi_version(void) { return FPF_ABI_VERSION; }

extern "C" const char* fpf_describe(void) {
  return "libfpf_hip abi 1: gfx950 HIP kernels for the pair-stack hot path -- layernorm, transition (LN + SwiGLU, "
         "bf16 MFMA 32x32x16 / fp32), trimul (K1 planes + batched MFMA contraction + K3), triattn (flash core with "
         "row-shared pair bias; prologue / epilogue block)";
}

extern "C" int fpf_layernorm_fwd(const FpfLnArgs* a, void* stream, char* err, size_t errlen) {
  using namespace fpf;
  FPF_CHECK_VERSION(a);
  if (!a->x || !a->y) return fail(err, errlen, FPF_E_ARGS, "x / y is NULL");
  if (a->rows < 0 || a->cols <= 0 || a->cols > 1024) return fail(err, errlen, FPF_E_SHAPE, "rows=%lld cols=%d", (long long)a->rows, a->cols);
  if (a->rows == 0) return FPF_OK;
  const bool in16 = a->dtype_in == FPF_DT_BF16, out16 = a->dtype_out == FPF_DT_BF16;
  if (!(in16 || a->dtype_in == FPF_DT_F32) || !(out16 || a->dtype_out == FPF_DT_F32))
    return fail(err, errlen, FPF_E_DTYPE, "dtype_in=%d dtype_out=%d", a->dtype_in, a->dtype_out);
  const int ein = in16 ? 8 : 4, eout = out16 ? 8 : 4;
  if (a->cols % ein || a->cols % eout || a->x_row_stride % ein || a->y_row_stride % eout || !aligned16(a->x) || !aligned16(a->y))
    return fail(err, errlen, FPF_E_ALIGN, "cols / row strides must be multiples of %d elements and x, y 16-byte aligned", ein);
  if (a->x_row_stride < a->cols || a->y_row_stride < a->cols) return fail(err, errlen, FPF_E_SHAPE, "row stride < cols");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (in16 && out16) return launch_ln<uint16_t, uint16_t>(a, st, err, errlen);
  if (in16) return launch_ln<uint16_t, float>(a, st, err, errlen);
  if (out16) return launch_ln<float, uint16_t>(a, st, err, errlen);
  return launch_ln<float, float>(a, st, err, errlen);
}
