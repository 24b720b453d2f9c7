// Shared device and host helpers of libfpf_hip.so (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "fpf_hip.h"

namespace fpf {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

// ---------------------------------------------------------------------------------------------------------------- bf16
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }  // RNE (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  bf16x2 r;
  r.x = (__bf16)a;
  r.y = (__bf16)b;
  return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ float lo_bf(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float hi_bf(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// ---------------------------------------------------------------------------------------------------------------- MFMA
// v_mfma_f32_32x32x16_bf16: A [32 x 16] lane l holds A[l%32][8*(l/32) .. +7]; B [16 x 32] lane l holds B[8*(l/32) .. +7][l%32];
// D [32 x 32] lane l, register v holds D[8*(v/4) + 4*(l/32) + v%4][l%32].
__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ bf16x8 as_bf8(const u32x4& u) { return __builtin_bit_cast(bf16x8, u); }
__device__ __forceinline__ int c_row(int v, int g) { return 8 * (v >> 2) + 4 * g + (v & 3); }   // D-layout row of register v

// ---------------------------------------------------------------------------------------------------------------- misc device
// Cross-half reductions of a wave64 (lanes l and l ^ 32) with v_permlane32_swap: after swapping x with itself, the two
// results hold {x[0..31], x[0..31]} and {x[32..63], x[32..63]}, so their sum / max is the pair's in every lane.
__device__ __forceinline__ float half_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float half_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
// acc + lo(p) + hi(p) for a packed bf16 pair (v_dot2_f32_bf16 against (1, 1))
__device__ __forceinline__ float dot2_bf16(uint32_t p, float acc) {
  const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, p), one, acc, false);
}
// bf16-path sigmoid / silu: v_exp_f32 + v_rcp_f32 (about 1 ulp each; the result is rounded to bf16 or feeds a bf16 MFMA)
__device__ __forceinline__ float sigmoidf_(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
__device__ __forceinline__ float siluf_(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
__device__ __forceinline__ float sigmoid_exact(float x) { return 1.0f / (1.0f + expf(-x)); }

template <typename T>
__device__ __forceinline__ T ldg(const T* p) { return __builtin_nontemporal_load(p); }

// ---------------------------------------------------------------------------------------------------------------- host
inline int fail(char* err, size_t errlen, int code, const char* fmt, ...) {
  if (err && errlen) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, errlen, fmt, ap);
    va_end(ap);
  }
  return code;
}

inline int launched(char* err, size_t errlen, const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(err, errlen, FPF_E_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return FPF_OK;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Compute units of the current device (queried once per device; sizes the persistent grids).
inline int num_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cache[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}
__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace fpf

#define FPF_CHECK_VERSION(a)                                                                                        \
  do {                                                                                                              \
    if (!(a)) return ::fpf::fail(err, errlen, FPF_E_ARGS, "null argument block");                                 \
    if ((a)->abi_version != FPF_ABI_VERSION)                                                                        \
      return ::fpf::fail(err, errlen, FPF_E_VERSION, "abi_version %d != %d", (int)(a)->abi_version, FPF_ABI_VERSION); \
  } while (0)
