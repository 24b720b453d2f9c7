// Triangle attention: the flash core (op) and the fused block (prologue -> core -> epilogue).
// Replaces common/opt_core/opt_core/kernels/triattn/__init__.py:1094 (triangle_attention, op :3-8) and
// common/opt_core/opt_core/attn/pair_fused.py:1500 (tri_attn_block; prologue :1136, core_attention :1391, epilogue :1416).
//
// bf16 core (head_dim 32): a workgroup = 4 waves x 32 queries of one (b, h) and R = 4 pair rows.  The per-key-tile bias tile
// (one per wave: its 32 queries x 32 keys) is loaded ONCE into registers and reused by all R rows; the R rows' K and V^T tiles
// are staged in LDS once and read by all 4 waves.  S^T = K Q^T is computed with v_mfma_f32_32x32x16_bf16 starting from the
// bias tile as the accumulator, so each lane owns ONE query and 16 of the 32 keys (the other 16 in lane ^ 32): the softmax
// max is 16 in-lane maxes + one cross-half exchange, the running sum stays per lane until the end, and P (bf16) is already
// the B operand of O^T = V^T P^T -- the key order inside a k-step is permuted identically in V^T.  exp2 with scale*log2(e)
// folded into one FMA.  A row whose keys are all masked attends uniformly to every key (the op's convention).
// fp32 core (exact tier): one thread per query, LDS-staged K / V tiles, fp32 online softmax with expf.
#include <algorithm>
#include <cmath>

#include "triattn.h"

namespace fpf {


// S^T tile of one pair row: keys of sub-tile `sub` (A = K rows from LDS) x this wave's 32 queries (B = Q^T), accumulated onto
// the bias tile.
__device__ __forceinline__ f32x16 qk_tile(const uint16_t* __restrict__ kr, int sub, int n, int g, const bf16x8 (&qf)[2], const f32x16& bt) {
  const uint16_t* row = kr + (32 * sub + n) * TA_KLD + 8 * g;
  f32x16 s = mfma32(as_bf8(*reinterpret_cast<const u32x4*>(row)), qf[0], bt);
  return mfma32(as_bf8(*reinterpret_cast<const u32x4*>(row + 16)), qf[1], s);
}

// VT: V stored transposed ([.., D, S]); BVEC: fp32 bias with 16-byte aligned rows (float4 loads; the generic variant reads
// element by element and serves bf16 or unaligned bias)
template <bool VT, bool BVEC>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) triattn_core_bf16(const CoreParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t sK[TA_R][TA_KT * TA_KLD];
  __shared__ __attribute__((aligned(16))) uint16_t sV[TA_R][TA_D * TA_VLD];
  __shared__ uint64_t sKeep[TA_R];
  __shared__ int sAlive[TA_R];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, n = l & 31, g = l >> 5;
  // logical work order (b h) -> row group -> query tile, dealt to the 8 XCDs in contiguous runs
  const int64_t nq = cdiv(p.S, 128), nr = cdiv(p.N, TA_R);
  const int64_t total = p.B * p.H * nr * nq;
  const int64_t per = (total + 7) / 8;
  const int64_t w = (blockIdx.x % 8) * per + blockIdx.x / 8;
  if (w >= total) return;
  const int64_t qt = w % nq, rg = (w / nq) % nr, bh = w / (nq * nr);
  const int64_t b = bh / p.H, h = bh % p.H;
  const int64_t i0 = rg * TA_R;
  const int64_t q = qt * 128 + wave * 32 + n;          // this lane's query
  const bool qlive = q < p.S;
  const float c2 = p.scale * LOG2E;                     // qk units -> log2 units
  const float inv_scale = 1.0f / p.scale;

  // this lane's Q fragments of the R rows (B operand of S^T = K Q^T: query q, d = 8g .. +7 and 16 + 8g .. +7), kept in
  // registers for the whole kernel; row liveness
  if (tid < TA_R) sAlive[tid] = 0;
  bf16x8 qf[TA_R][2];
#pragma unroll
  for (int r = 0; r < TA_R; ++r) {
    const int64_t i = i0 + r;
    const bool ok = i < p.N && qlive;
    const uint16_t* qp = p.q + b * p.qs[0] + (ok ? i : 0) * p.qs[1] + h * p.qs[2] + (ok ? q : 0) * p.qs[3] + 8 * g;
    qf[r][0] = as_bf8(ok ? *reinterpret_cast<const u32x4*>(qp) : u32x4{0, 0, 0, 0});
    qf[r][1] = as_bf8(ok ? *reinterpret_cast<const u32x4*>(qp + 16) : u32x4{0, 0, 0, 0});
  }
  __syncthreads();
  for (int r = 0; r < TA_R; ++r) {
    const int64_t i = i0 + r;
    if (i >= p.N) continue;
    int any = 0;
    for (int64_t key = tid; key < p.S && !any; key += 256) any = mask_keep(p, b, i, key);
    if (any) sAlive[r] = 1;
  }
  __syncthreads();
  bool dead[TA_R];
  bool dead_any = false;
#pragma unroll
  for (int r = 0; r < TA_R; ++r) {
    dead[r] = (i0 + r < p.N) && !sAlive[r];
    dead_any |= dead[r];
  }
  const bool wave_row_dead = wave < TA_R ? !sAlive[wave] : true;

  f32x16 o[TA_R];
  float mrow[TA_R], lrow[TA_R];                         // running max (log2 units) and this lane's partial sum
#pragma unroll
  for (int r = 0; r < TA_R; ++r) {
    o[r] = f32x16{};
    mrow[r] = -INFINITY;
    lrow[r] = 0.f;
  }

  // staging: 1024 16-byte chunks per operand per tile, 4 per thread; element offsets at key 0 are computed once
  // chunk `it` of a thread belongs to row i0 + it (256 threads x 4 chunks): row bases are wave-uniform, the in-row part per lane
  // row base pointers are wave-uniform (scalar registers); the in-row part is one 32-bit per-lane offset per operand
  const uint16_t* kbase[TA_R];
  const uint16_t* vbase[TA_R];
  bool rowok[TA_R];
#pragma unroll
  for (int it = 0; it < TA_R; ++it) {
    const int64_t i = i0 + it;
    rowok[it] = i < p.N;
    const int64_t ii = rowok[it] ? i : i0;
    kbase[it] = p.k + b * p.ks[0] + ii * p.ks[1] + h * p.ks[2];
    vbase[it] = p.v + b * p.vs[0] + ii * p.vs[1] + h * p.vs[2];
  }
  const uint32_t kin = (uint32_t)(((tid >> 2) & 63) * p.ks[3] + 8 * (tid & 3));
  const uint32_t vin = (uint32_t)(VT ? ((tid >> 3) & 31) * p.vs[3] + 8 * (tid & 7) : ((tid >> 2) & 63) * p.vs[3] + 8 * (tid & 3));
  u32x4 rk[TA_R], rv[TA_R];
  bool keepn;                                           // prefetched mask bit: row i0 + wave, key k0 + l of the next tile
  auto gload = [&](int64_t k0) {
    {
      const int64_t i = i0 + wave, key = k0 + l;
      keepn = wave < TA_R && key < p.S && i < p.N && (wave_row_dead || mask_keep(p, b, i, key));
    }
    if (k0 + TA_KT <= p.S) {                              // whole tile in range (uniform)
#pragma unroll
      for (int it = 0; it < TA_R; ++it) {
        rk[it] = rowok[it] ? *reinterpret_cast<const u32x4*>(kbase[it] + k0 * p.ks[3] + kin) : u32x4{0, 0, 0, 0};
        rv[it] = rowok[it] ? *reinterpret_cast<const u32x4*>(vbase[it] + (VT ? k0 : k0 * p.vs[3]) + vin) : u32x4{0, 0, 0, 0};
      }
      return;
    }
#pragma unroll
    for (int it = 0; it < TA_R; ++it) {
      const int c = tid + 256 * it;
      const int64_t kkey = k0 + ((c >> 2) & 63);
      rk[it] = (rowok[it] && kkey < p.S) ? *reinterpret_cast<const u32x4*>(kbase[it] + k0 * p.ks[3] + kin) : u32x4{0, 0, 0, 0};
      if constexpr (VT) {
        const int64_t key = k0 + 8 * (c & 7);
        const uint16_t* src = vbase[it] + k0 + vin;
        uint16_t tmp[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) tmp[e] = (rowok[it] && key + e < p.S) ? src[e] : (uint16_t)0;
        rv[it] = u32x4{tmp[0] | ((uint32_t)tmp[1] << 16), tmp[2] | ((uint32_t)tmp[3] << 16), tmp[4] | ((uint32_t)tmp[5] << 16),
                       tmp[6] | ((uint32_t)tmp[7] << 16)};
      } else {
        rv[it] = (rowok[it] && kkey < p.S) ? *reinterpret_cast<const u32x4*>(vbase[it] + k0 * p.vs[3] + vin) : u32x4{0, 0, 0, 0};
      }
    }
  };
  // bias of one 32-key sub-tile (raw values, keys kb + 8 qd + 4 g + 0..3), prefetched one sub-tile ahead
  const int64_t bias_row = b * p.bs[0] + h * p.bs[1] + (qlive ? q : 0) * p.bs[2];
  auto bload = [&](int64_t kb, f32x16& dst) {
    const int64_t kb0 = kb + 4 * g;
    if constexpr (BVEC) {                           // S % 4 == 0: a 4-key chunk lies wholly below S or wholly past it
      const float* bp = static_cast<const float*>(p.bias) + bias_row;
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int64_t k4 = kb0 + 8 * qd;
        const f32x4 v4 = k4 < p.S ? *reinterpret_cast<const f32x4*>(bp + k4) : f32x4{0.f, 0.f, 0.f, 0.f};   // past S: masked keys
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[4 * qd + e] = v4[e];
      }
    } else {
#pragma unroll
      for (int qd = 0; qd < 4; ++qd)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t key = kb0 + 8 * qd + e;
          dst[4 * qd + e] = key < p.S ? bias_at(p, bias_row + key * p.bs[3]) : 0.f;
        }
    }
  };

  gload(0);
  f32x16 bnext;
  bload(0, bnext);
  for (int64_t k0 = 0; k0 < p.S; k0 += TA_KT) {
    __syncthreads();
#pragma unroll
    for (int it = 0; it < TA_R; ++it) {
      const int c = tid + 256 * it;
      const int r = c >> 8;
      *reinterpret_cast<u32x4*>(&sK[r][((c >> 2) & 63) * TA_KLD + 8 * (c & 3)]) = rk[it];
      if constexpr (VT) {
        uint16_t* dst = &sV[r][((c >> 3) & 31) * TA_VLD + 8 * (c & 7)];
        *reinterpret_cast<u32x2*>(dst) = u32x2{rv[it][0], rv[it][1]};
        *reinterpret_cast<u32x2*>(dst + 4) = u32x2{rv[it][2], rv[it][3]};
      } else {
        const int kk = (c >> 2) & 63, part = c & 3;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sV[r][(8 * part + 2 * e) * TA_VLD + kk] = (uint16_t)(rv[it][e] & 0xffff);
          sV[r][(8 * part + 2 * e + 1) * TA_VLD + kk] = (uint16_t)(rv[it][e] >> 16);
        }
      }
    }
    {
      const uint64_t bal = __ballot(keepn);               // keep bits of row `wave`: lane l <-> key k0 + l
      if (l == 0 && wave < TA_R) sKeep[wave] = bal;
    }
    __syncthreads();
    if (k0 + TA_KT < p.S) gload(k0 + TA_KT);
    uint64_t kall = ~0ull, kany = 0;
#pragma unroll
    for (int r = 0; r < TA_R; ++r) {
      kall &= sKeep[r];
      kany |= sKeep[r];
    }
    const bool full = (kall == ~0ull) && !dead_any;       // uniform: no masking work in this tile
#pragma unroll 1
    for (int sub = 0; sub < 2; ++sub) {
      f32x16 bt;
#pragma unroll
      for (int v = 0; v < 16; ++v) bt[v] = bnext[v] * inv_scale;      // qk units: the accumulator's initial value
      {
        const int64_t kn = sub == 0 ? k0 + 32 : k0 + TA_KT;             // prefetch the next sub-tile's bias
        if (kn < p.S) bload(kn, bnext);
      }
      if ((uint32_t)(kany >> (32 * sub)) == 0) continue;               // no row keeps a key of this sub-tile
      f32x16 s[TA_R];
#pragma unroll
      for (int r = 0; r < TA_R; ++r) {
        s[r] = qk_tile(sK[r], sub, n, g, qf[r], bt);
      }
      if (!full) {
#pragma unroll
        for (int r = 0; r < TA_R; ++r) {
          const uint32_t kb = (uint32_t)(sKeep[r] >> (32 * sub));
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const float sv = dead[r] ? 0.f : s[r][v];
            s[r][v] = ((kb >> c_row(v, g)) & 1u) ? sv : -INFINITY;
          }
        }
      }
      float mx[TA_R];
      bool need = false;
#pragma unroll
      for (int r = 0; r < TA_R; ++r) {
        float m0 = s[r][0];                      // a linear chain: the compiler folds it into v_max3_f32
#pragma unroll
        for (int v = 1; v < 16; ++v) m0 = fmaxf(m0, s[r][v]);
        mx[r] = half_max(m0) * c2;
        need |= mx[r] > mrow[r] + TA_HEADROOM;
      }
      if (__ballot(need) != 0) {       // some query's max moved past the headroom: move that query's running max (exact)
#pragma unroll
        for (int r = 0; r < TA_R; ++r) {
          // per lane and row: a query's trajectory depends on its own logits only, so results do not depend on which rows
          // share a workgroup (row-chunked calls are bitwise equal to whole-tensor ones)
          const float mnew = (mx[r] > mrow[r] + TA_HEADROOM) ? fmaxf(mrow[r], mx[r]) : mrow[r];
          const float alpha = (mnew == -INFINITY) ? 1.0f : fast_exp2(mrow[r] - mnew);
          lrow[r] *= alpha;
#pragma unroll
          for (int v = 0; v < 16; ++v) o[r][v] *= alpha;
          mrow[r] = mnew;
        }
      }
#pragma unroll
      for (int r = 0; r < TA_R; ++r) {
        const float mb = (mrow[r] == -INFINITY) ? 0.f : mrow[r];
        uint32_t pk[8];
        float ps0 = lrow[r], ps1 = 0.f;
#pragma unroll
        for (int v = 0; v < 16; v += 2) {
          const float p0 = fast_exp2(fmaf(s[r][v], c2, -mb));
          const float p1 = fast_exp2(fmaf(s[r][v + 1], c2, -mb));
          pk[v >> 1] = pack2(p0, p1);
          if (v & 2) ps1 = dot2_bf16(pk[v >> 1], ps1);      // the row sum of the bf16 P the PV MFMA consumes
          else ps0 = dot2_bf16(pk[v >> 1], ps0);
        }
        lrow[r] = ps0 + ps1;
        const uint16_t* vr = sV[r] + n * TA_VLD + 32 * sub + 4 * g;
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const u32x2 lo = *reinterpret_cast<const u32x2*>(vr + 16 * st);
          const u32x2 hi = *reinterpret_cast<const u32x2*>(vr + 16 * st + 8);
          o[r] = mfma32(as_bf8(u32x4{lo[0], lo[1], hi[0], hi[1]}), as_bf8(u32x4{pk[4 * st], pk[4 * st + 1], pk[4 * st + 2], pk[4 * st + 3]}), o[r]);
        }
      }
    }
  }
  if (!qlive) return;
#pragma unroll
  for (int r = 0; r < TA_R; ++r) {
    const int64_t i = i0 + r;
    if (i >= p.N) continue;
    const float lt = half_sum(lrow[r]);
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    uint16_t* op = p.out + b * p.os[0] + i * p.os[1] + h * p.os[2] + q * p.os[3];
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const int d0 = 8 * qd + 4 * g;
      *reinterpret_cast<u32x2*>(op + d0) = u32x2{pack2(o[r][4 * qd] * inv, o[r][4 * qd + 1] * inv), pack2(o[r][4 * qd + 2] * inv, o[r][4 * qd + 3] * inv)};
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------- fp32 core
struct CoreParamsF {
  const float* q;
  const float* k;
  const float* v;
  int64_t qs[5], ks[5], vs[5];
  const void* bias;
  int bias_bf16;
  int64_t bs[4];
  const void* mask;
  int mask_f32;
  int64_t ms[3];
  float* out;
  int64_t os[5];
  int64_t B, N, H, S;
  float scale;
};

constexpr int TF_QT = 64;   // queries per workgroup (one per thread)
constexpr int TF_KT = 32;

template <int D>
__global__ void __launch_bounds__(64) triattn_core_f32(const CoreParamsF p) {
  __shared__ float sK[TF_KT][D + 1];
  __shared__ float sV[TF_KT][D + 1];
  __shared__ int sKeep[TF_KT];
  __shared__ int sAlive;
  const int tid = threadIdx.x;
  const int64_t nq = cdiv(p.S, TF_QT);
  const int64_t qt = blockIdx.x % nq, rest = blockIdx.x / nq;
  const int64_t h = rest % p.H, i = (rest / p.H) % p.N, b = rest / (p.H * p.N);
  const int64_t q = qt * TF_QT + tid;
  const bool qlive = q < p.S;
  if (tid == 0) sAlive = 0;
  __syncthreads();
  {
    int any = 0;
    for (int64_t key = tid; key < p.S && !any; key += TF_QT) {
      if (!p.mask) { any = 1; break; }
      const int64_t off = b * p.ms[0] + i * p.ms[1] + key * p.ms[2];
      any = p.mask_f32 ? (static_cast<const float*>(p.mask)[off] != 0.f) : (static_cast<const uint8_t*>(p.mask)[off] != 0);
    }
    if (any) atomicOr(&sAlive, 1);
  }
  __syncthreads();
  const bool dead = !sAlive;
  float qv[D], ov[D];
  const float* qp = p.q + b * p.qs[0] + i * p.qs[1] + h * p.qs[2] + q * p.qs[3];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    qv[d] = qlive ? qp[d] : 0.f;
    ov[d] = 0.f;
  }
  float m = -INFINITY, lsum = 0.f;
  for (int64_t k0 = 0; k0 < p.S; k0 += TF_KT) {
    __syncthreads();
    for (int c = tid; c < TF_KT * D; c += TF_QT) {
      const int kk = c / D, d = c % D;
      const int64_t key = k0 + kk;
      const bool ok = key < p.S;
      sK[kk][d] = ok ? p.k[b * p.ks[0] + i * p.ks[1] + h * p.ks[2] + key * p.ks[3] + d] : 0.f;
      sV[kk][d] = ok ? p.v[b * p.vs[0] + i * p.vs[1] + h * p.vs[2] + key * p.vs[3] + d] : 0.f;
    }
    if (tid < TF_KT) {
      const int64_t key = k0 + tid;
      bool keep = key < p.S;
      if (keep && !dead && p.mask) {
        const int64_t off = b * p.ms[0] + i * p.ms[1] + key * p.ms[2];
        keep = p.mask_f32 ? (static_cast<const float*>(p.mask)[off] != 0.f) : (static_cast<const uint8_t*>(p.mask)[off] != 0);
      }
      sKeep[tid] = keep;
    }
    __syncthreads();
    float sc[TF_KT];
    float tmax = -INFINITY;
#pragma unroll
    for (int kk = 0; kk < TF_KT; ++kk) {
      float s = -INFINITY;
      if (sKeep[kk]) {
        if (dead) {
          s = 0.f;
        } else {
          float dot = 0.f;
#pragma unroll
          for (int d = 0; d < D; ++d) dot = fmaf(qv[d], sK[kk][d], dot);
          const int64_t key = k0 + kk;
          const float bb = qlive ? (p.bias_bf16 ? bf2f(static_cast<const uint16_t*>(p.bias)[b * p.bs[0] + h * p.bs[1] + q * p.bs[2] + key * p.bs[3]])
                                                : static_cast<const float*>(p.bias)[b * p.bs[0] + h * p.bs[1] + q * p.bs[2] + key * p.bs[3]])
                                 : 0.f;
          s = dot * p.scale + bb;
        }
      }
      sc[kk] = s;
      tmax = fmaxf(tmax, s);
    }
    if (tmax == -INFINITY) continue;
    const float mnew = fmaxf(m, tmax);
    const float alpha = expf(m - mnew);
    lsum *= alpha;
#pragma unroll
    for (int d = 0; d < D; ++d) ov[d] *= alpha;
#pragma unroll
    for (int kk = 0; kk < TF_KT; ++kk) {
      const float pe = expf(sc[kk] - mnew);
      lsum += pe;
#pragma unroll
      for (int d = 0; d < D; ++d) ov[d] = fmaf(pe, sV[kk][d], ov[d]);
    }
    m = mnew;
  }
  if (!qlive) return;
  const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
  float* op = p.out + b * p.os[0] + i * p.os[1] + h * p.os[2] + q * p.os[3];
#pragma unroll
  for (int d = 0; d < D; ++d) op[d] = ov[d] * inv;
}

// ---------------------------------------------------------------------------------------------------------------- prologue (bf16)
// x = LN(z or z^T) -> q, k [B,I,H,J,D] bf16, v^T [B,I,H,D,Jp] bf16 (Jp = N rounded up to 32; the core stages V^T rows
// directly), g [B,I,J,HD] bf16 (pre-sigmoid), bias [B,H,I,J] fp32.  Every bf16 output leaves in 16-byte stores.  Persistent: W_qkvg (512 rows) and W_b (padded to 32 rows) live in LDS (148 KB); a wave
// owns 32 positions j of one attention row i; with `ending` the 32 z pixels are z[j][i] (strided rows, each a contiguous
// 256-byte pixel).
constexpr int TP_C = 128, TP_HD = 128;

// Outputs are selected by flags (PRO_QKV: q, k, v^T; PRO_G: g; PRO_BIAS: the full bias) and cover the attention rows
// [row0, row0 + rows): q / k / v^T / g are indexed by the row within that range, the bias by the absolute row.  The `big`
// chunked driver runs a bias-only pass over every row, then q / k / v^T per row chunk.
enum { PRO_QKV = 1, PRO_G = 2, PRO_BIAS = 4, PRO_VPERM = 8, PRO_BIAS_BLK = 16 };  // VPERM: V^T keys in the core's 16-block
// order; BIAS_BLK: the bias planes in the block-layout core's 32 x 32 register-order blocks (bias_blk_off; fp32, N % 32 == 0)
struct ProParams {
  const uint16_t* z;
  const float* ln_w;
  const float* ln_b;
  float eps;
  const uint16_t* w_qkvg;
  const uint16_t* w_b;
  int H;
  uint16_t* q;
  uint16_t* k;
  uint16_t* v;
  uint16_t* g;
  float* bias;
  int64_t N, Jp, B, row0, rows;
  int ending, flags;
  float q_scale;                 // q is stored times this (the fused block folds the attention scale into q)
  float bias_scale;              // and the bias times this (log2(e) for the block-layout core: logits in log2 units)
  int64_t bias_ld;               // elements between bias rows (>= N)
  int bias_bf16;                 // bias stored as bf16 (else fp32)
  const float* b_g;              // [HD] gate projection bias added to g, or NULL
  const uint16_t* xln;           // the caller's LayerNorm output [B, N, N, 128] bf16 in the attention frame (XLN instance), or NULL
  int64_t Np;                    // J extent of the q / k rows and of the blocked bias planes: N, or N padded to 64 for the
                                 // block-layout core (then every 32-pixel tile up to Np is computed, so V^T's padding keys hold
                                 // finite values; the padding rows of q / k and of the bias are never written)
};

// XLN: the rows come from p.xln (the caller's own LayerNorm output, attention frame) and are projected as they are.
template <bool XLN>
__global__ void __launch_bounds__(512) triattn_prologue_bf16(const ProParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t sW[(4 * TP_HD + 32) * RT_LD];
  __shared__ __attribute__((aligned(16))) float sLN[2 * RT_C];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  rt_stage_affine(sLN, p.ln_w, p.ln_b, tid, 512);
  if (p.flags & (PRO_QKV | PRO_G)) rt_stage_weights(sW, p.w_qkvg, 4 * TP_HD, 4 * TP_HD, tid, 512);
  rt_stage_weights(sW + 4 * TP_HD * RT_LD, p.w_b, 32, p.H, tid, 512);
  __syncthreads();
  const int H = p.H, D = TP_HD / H;
  const int64_t N = p.N, Jp = p.Jp, R = p.rows, Np = p.Np;
  const uint32_t tpr = (uint32_t)cdiv(Np, 32), per_b = (uint32_t)R * tpr, total = (uint32_t)p.B * per_b;
  const uint32_t stride = gridDim.x * RT_WAVES;
  u32x4 raw[8];                                         // the next tile's pixel rows, loaded while this tile computes
  // the lane index is re-read per tile (opaque_lane): lane-dependent address parts kept live across the tile loop would
  // be spilled, and each reload's wait would also drain the next tile's prefetch
  auto fetch = [&](uint32_t tt) {
    const int ln = opaque_lane(), n = ln & 31, g = ln >> 5;
    const RtTile tl = rt_tile(tt, per_b, tpr);
    const int64_t b = tl.b, i = p.row0 + tl.r, j = tl.c * 32 + n;
    const bool live = j < N;
    if constexpr (XLN) {
      rt_load(p.xln + ((b * N + i) * N + (live ? j : 0)) * RT_C, live, g, raw);
    } else {
      const int64_t zpix = p.ending ? (b * N + (live ? j : 0)) * N + i : (b * N + i) * N + (live ? j : 0);
      rt_load(p.z + zpix * RT_C, live, g, raw);
    }
  };
  if (blockIdx.x * RT_WAVES + wave < total) fetch(blockIdx.x * RT_WAVES + wave);
  for (uint32_t t = blockIdx.x * RT_WAVES + wave; t < total; t += stride) {
    const int ln = opaque_lane(), n = ln & 31, g = ln >> 5;
    const RtTile tl = rt_tile(t, per_b, tpr);
    const int64_t b = tl.b, ii = tl.r, i = p.row0 + ii, j = tl.c * 32 + n;
    const bool live = j < N;
    bf16x8 xb[8];
    if constexpr (XLN) {
#pragma unroll
      for (int c = 0; c < 8; ++c) xb[c] = as_bf8(raw[c]);
    } else {
      rt_ln(raw, g, sLN, p.eps, xb);
    }
    if (t + stride < total) fetch(t + stride);
    // two output blocks per iteration: the second block's MFMA chain is issued while the first one's results are packed and
    // stored (one block at a time left the matrix core idle during each store phase: 156 -> 148 us at N = 768)
#pragma unroll 2
    for (int blk = 0; blk < 17; ++blk) {
      if (blk < 12 && !(p.flags & PRO_QKV)) continue;
      if (blk >= 12 && blk < 16 && !(p.flags & PRO_G)) continue;
      if (blk == 16 && !(p.flags & PRO_BIAS)) continue;
      if (blk >= 8 && blk < 12) {                         // v, transposed: vT[b][ii][h][d][Jp] -- the swapped product x W_v^T
        // puts d on the lanes and 16 pixels in the registers; the lane exchange then gives each lane 8 consecutive pixels
        const f32x16 acc = rt_gemm32_xw(sW, blk * 32, n, g, xb);
        u32x4 lo, hi;
        if (p.flags & PRO_VPERM) {                        // keys of each 16-block as {0-3, 8-11 | 4-7, 12-15}: the lane's
          lo = u32x4{pack2(acc[0], acc[1]), pack2(acc[2], acc[3]), pack2(acc[4], acc[5]), pack2(acc[6], acc[7])};   // D-layout
          hi = u32x4{pack2(acc[8], acc[9]), pack2(acc[10], acc[11]), pack2(acc[12], acc[13]), pack2(acc[14], acc[15])};  // rows
        } else {
          rt_pack16(acc, lo, hi);
        }
        uint16_t* dst = p.v + (((b * R + ii) * H + (blk & 3)) * (int64_t)D + n) * Jp + (j - n) + 8 * g;
        *reinterpret_cast<u32x4*>(dst) = lo;               // whole 32-pixel tile: Jp covers it (padding is never read)
        *reinterpret_cast<u32x4*>(dst + 16) = hi;
        continue;
      }
      f32x16 acc = rt_gemm32(sW, blk * 32, n, g, xb);
      if (blk < 4 && p.q_scale != 1.0f) acc *= p.q_scale;
      if (blk >= 12 && blk < 16 && p.b_g) {
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[v] += p.b_g[(blk - 12) * 32 + c_row(v, g)];
      }
      if (blk < 16) {                                     // q | k | g
        u32x4 lo, hi;
        rt_pack16(acc, lo, hi);
        if (!live) continue;
        uint16_t* dst = blk < 8 ? (blk < 4 ? p.q : p.k) + (((b * R + ii) * H + (blk & 3)) * Np + j) * D + 8 * g  // [B, R, H, Np, D]
                                : p.g + ((b * R + ii) * N + j) * TP_HD + (blk - 12) * 32 + 8 * g;             // [B, R, J, HD]
        *reinterpret_cast<u32x4*>(dst) = lo;
        *reinterpret_cast<u32x4*>(dst + 16) = hi;
      } else if (live) {                                  // bias: [B, H, I, bias_ld] fp32 | bf16, absolute row; head c_row(v, g)
        const bool blk_bias = (p.flags & PRO_BIAS_BLK) != 0;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int hh = c_row(v, g);
          if (hh >= H) continue;
          const int64_t o = blk_bias ? (b * H + hh) * Np * Np + bias_blk_off(Np, i, j) : ((b * H + hh) * N + i) * p.bias_ld + j;
          if (p.bias_bf16) reinterpret_cast<uint16_t*>(p.bias)[o] = f2bf(acc[v] * p.bias_scale);
          else p.bias[o] = acc[v] * p.bias_scale;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------- epilogue (bf16)
// u = (sigmoid(g) * o) W_o^T; residual: z[i,j] += u (ending: z[j,i] += u) in place; else out[zpix] = u.  Persistent: W_o lives in
// LDS; a wave owns 32 positions of one attention row.
__global__ void __launch_bounds__(512) triattn_epilogue_bf16(const uint16_t* __restrict__ o, const uint16_t* __restrict__ gt,
                                                             const uint16_t* __restrict__ w_o, const float* __restrict__ b_o, int H, uint16_t* zout,
                                                             int64_t N, int64_t B, int ending, int residual) {
  __shared__ __attribute__((aligned(16))) uint16_t sW[RT_C * RT_LD];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, n = l & 31, g = l >> 5;
  rt_stage_weights(sW, w_o, RT_C, RT_C, tid, 512);
  __syncthreads();
  const int D = TP_HD / H;
  const uint32_t tpr = (uint32_t)cdiv(N, 32), per_b = (uint32_t)N * tpr, total = (uint32_t)B * per_b;
  const uint32_t stride = gridDim.x * RT_WAVES;
  for (uint32_t t = blockIdx.x * RT_WAVES + wave; t < total; t += stride) {
    const RtTile tl = rt_tile(t, per_b, tpr);
    const int64_t b = tl.b, i = tl.r, j = tl.c * 32 + n;
    const bool live = j < N;
    bf16x8 xb[8];
#pragma unroll
    for (int tt = 0; tt < 8; ++tt) {
      const int hd0 = 8 * rt_chunk(tt, g);
      const int hh = hd0 / D, d0 = hd0 % D;
      u32x4 ov = {0, 0, 0, 0}, gv = {0, 0, 0, 0};
      if (live) {
        ov = *reinterpret_cast<const u32x4*>(o + (((b * N + i) * H + hh) * N + j) * D + d0);
        gv = *reinterpret_cast<const u32x4*>(gt + ((b * N + i) * N + j) * TP_HD + hd0);
      }
      uint32_t w4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) w4[e] = pack2(sigmoidf_(lo_bf(gv[e])) * lo_bf(ov[e]), sigmoidf_(hi_bf(gv[e])) * hi_bf(ov[e]));
      xb[tt] = as_bf8(u32x4{w4[0], w4[1], w4[2], w4[3]});
    }
    const int64_t zpix = ending ? (b * N + j) * N + i : (b * N + i) * N + j;
    uint16_t* zp = zout + zpix * RT_C + 8 * g;
#pragma unroll 1
    for (int cb = 0; cb < 4; ++cb) {
      f32x16 acc = rt_gemm32(sW, cb * 32, n, g, xb);
      if (b_o) {
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[v] += b_o[cb * 32 + c_row(v, g)];
      }
      // lane (n, g) stores channels cb*32 + 8g .. +7 and cb*32 + 16 + 8g .. +7 of pixel n: two 16-byte stores
      if (residual) {
        float y[16];
        rt_regroup_f32(acc, y);
        if (!live) continue;
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          uint16_t* p = zp + cb * 32 + 16 * h2;
          const u32x4 r = *reinterpret_cast<const u32x4*>(p);
          u32x4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = pack2(y[8 * h2 + 2 * e] + lo_bf(r[e]), y[8 * h2 + 2 * e + 1] + hi_bf(r[e]));
          *reinterpret_cast<u32x4*>(p) = w;
        }
      } else {
        u32x4 lo, hi;
        rt_pack16(acc, lo, hi);
        if (!live) continue;
        *reinterpret_cast<u32x4*>(zp + cb * 32) = lo;
        *reinterpret_cast<u32x4*>(zp + cb * 32 + 16) = hi;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------- gate-fused epilogue (bf16)
// The block's epilogue without the g round trip: the gate is recomputed from the block's own input, g = LN(x) W_g^T (x = z
// or z^T, the pixel this wave updates anyway), so the prologue never writes g (151 MB at N = 768) and this kernel never
// reads it back.  u = (sigmoid(g) * o) W_o^T; residual: z += u in place (the LN input is read before the pixel is written,
// by the same lane).  The g GEMM's output fragments are used directly as the B operand of the W_o GEMM: k-step s = 2 cb +
// half takes, in lane half g, the channels cb*32 + 16 half + {4g .. 4g+3, 8+4g .. 8+4g+3} that the D layout leaves there,
// and W_o's columns are permuted identically when staged.
// XLN: the gate's input rows come from xln (the caller's LayerNorm output, attention frame) as they are; the residual reads z.
template <bool XLN>
__global__ void __launch_bounds__(512) triattn_epilogue_gate_bf16(const uint16_t* zin, const uint16_t* __restrict__ o,
                                                                  const float* __restrict__ ln_w, const float* __restrict__ ln_b, float eps,
                                                                  const uint16_t* __restrict__ w_g, const uint16_t* __restrict__ w_o,
                                                                  const float* __restrict__ b_g, const float* __restrict__ b_o,
                                                                  uint16_t* zout, int64_t N, int64_t B, int64_t row0, int64_t rows, int ending,
                                                                  int residual, int64_t Jo, const uint16_t* __restrict__ xln) {
  __shared__ __attribute__((aligned(16))) uint16_t sWg[RT_C * RT_LD];
  __shared__ __attribute__((aligned(16))) uint16_t sWo[RT_C * RT_LD];   // columns permuted to the k-step order above
  __shared__ __attribute__((aligned(16))) float sLN[2 * RT_C];
  __shared__ __attribute__((aligned(16))) float sBias[2 * RT_C];        // [b_g 128 | b_o 128] (zeros when absent)
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, n = l & 31, g = l >> 5;
  rt_stage_affine(sLN, ln_w, ln_b, tid, 512);
  const bool has_bg = b_g != nullptr, has_bo = b_o != nullptr;
  for (int i = tid; i < 2 * RT_C; i += 512) sBias[i] = i < RT_C ? (has_bg ? b_g[i] : 0.f) : (has_bo ? b_o[i - RT_C] : 0.f);
  rt_stage_weights(sWg, w_g, RT_C, RT_C, tid, 512);
  for (int q = tid; q < RT_C * RT_C; q += 512) {
    const int m = q >> 7, kp = q & 127;
    const int st = kp >> 4, gg = (kp >> 3) & 1, e = kp & 7;
    const int c = (st >> 1) * 32 + 16 * (st & 1) + 8 * (e >> 2) + 4 * gg + (e & 3);
    sWo[m * RT_LD + kp] = w_o[m * RT_C + c];
  }
  __syncthreads();
  constexpr int H = TP_HD / TA_D;
  const uint32_t tpr = (uint32_t)cdiv(N, 32), per_b = (uint32_t)rows * tpr, total = (uint32_t)B * per_b;
  const uint32_t stride = gridDim.x * RT_WAVES;
  // z rows of a tile: lane (n, g) chunk t holds channels 16t + 8g .. +7, exactly the channels its output stores cover, so the
  // residual reuses them; the next tile's rows are loaded while this tile computes
  u32x4 raw[8];
  auto zpix_of = [&](uint32_t tt, bool& live) {
    const RtTile tl = rt_tile(tt, per_b, tpr);
    const int64_t b = tl.b, i = row0 + tl.r, j = tl.c * 32 + n;
    live = j < N;
    return ending ? (b * N + (live ? j : 0)) * N + i : (b * N + i) * N + (live ? j : 0);
  };
  // the rows the gate reads: z (its LayerNorm is taken here), or the caller's x_ln at the attention-frame pixel
  auto in_rows = [&](uint32_t tt) {
    bool lv;
    const int64_t zp = zpix_of(tt, lv);
    if constexpr (XLN) {
      const RtTile tl = rt_tile(tt, per_b, tpr);
      const int64_t j = tl.c * 32 + n;
      rt_load(xln + ((tl.b * N + row0 + tl.r) * N + (lv ? j : 0)) * RT_C, lv, g, raw);
    } else {
      rt_load(zin + zp * RT_C, lv, g, raw);
    }
  };
  if (blockIdx.x * RT_WAVES + wave < total) in_rows(blockIdx.x * RT_WAVES + wave);
  for (uint32_t t = blockIdx.x * RT_WAVES + wave; t < total; t += stride) {
    const RtTile tl = rt_tile(t, per_b, tpr);
    const int64_t b = tl.b, ii = tl.r, j = tl.c * 32 + n;
    bool live;
    const int64_t zpix = zpix_of(t, live);
    // o of all four heads for this tile, issued before the LayerNorm
    u32x2 ov2[4][2][2];
    const uint16_t* op = o + (((b * rows + ii) * H) * Jo + (live ? j : 0)) * TA_D + 4 * g;   // o rows of this range (J extent Jo)
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
      for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int e = 0; e < 2; ++e)
          ov2[cb][half][e] = live ? *reinterpret_cast<const u32x2*>(op + (int64_t)cb * Jo * TA_D + 16 * half + 8 * e) : u32x2{0, 0};
    bf16x8 xb[8];
    if constexpr (XLN) {
#pragma unroll
      for (int c = 0; c < 8; ++c) xb[c] = as_bf8(raw[c]);
    } else {
      rt_ln(raw, g, sLN, eps, xb);
    }
    f32x16 acc[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) acc[k] = f32x16{};
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      f32x16 gacc = rt_gemm32_la<1>(sWg, cb * 32, n, g, xb);         // g of head cb: channels cb*32 + c_row(v, g)
      if (has_bg) {
#pragma unroll
        for (int v = 0; v < 16; ++v) gacc[v] += sBias[cb * 32 + c_row(v, g)];
      }
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const u32x2 o0 = ov2[cb][half][0], o1 = ov2[cb][half][1];
        const float ov[8] = {lo_bf(o0[0]), hi_bf(o0[0]), lo_bf(o0[1]), hi_bf(o0[1]), lo_bf(o1[0]), hi_bf(o1[0]), lo_bf(o1[1]), hi_bf(o1[1])};
        uint32_t w4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w4[e] = pack2(sigmoidf_(gacc[8 * half + 2 * e]) * ov[2 * e], sigmoidf_(gacc[8 * half + 2 * e + 1]) * ov[2 * e + 1]);
        const bf16x8 bop = as_bf8(u32x4{w4[0], w4[1], w4[2], w4[3]});
        const int kst = 2 * cb + half;
#pragma unroll
        for (int blk = 0; blk < 4; ++blk)
          acc[blk] = mfma32(as_bf8(*reinterpret_cast<const u32x4*>(&sWo[(blk * 32 + n) * RT_LD + 16 * kst + 8 * g])), bop, acc[blk]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // lane (n, g) stores channels blk*32 + 8g .. +7 and blk*32 + 16 + 8g .. +7 of pixel n: two 16-byte stores per block
    uint16_t* zp = zout + zpix * RT_C + 8 * g;
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      float y[16];
      rt_regroup_f32(acc[blk], y);
      if (!live) continue;
      if (has_bo) {                                                // y[8 h2 + e] is channel blk*32 + 16 h2 + 8g + e
#pragma unroll
        for (int e = 0; e < 16; ++e) y[e] += sBias[RT_C + blk * 32 + 16 * (e >> 3) + 8 * g + (e & 7)];
      }
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        u32x4 w;
        if (residual) {
          // channels blk*32 + 16 h2 + 8g .. +7 of this pixel: the z rows already held, or (x_ln read) z itself, read by the lane
          // that writes it
          const u32x4 r = XLN ? *reinterpret_cast<const u32x4*>(zin + zpix * RT_C + blk * 32 + 16 * h2 + 8 * g) : raw[2 * blk + h2];
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = pack2(y[8 * h2 + 2 * e] + lo_bf(r[e]), y[8 * h2 + 2 * e + 1] + hi_bf(r[e]));
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = pack2(y[8 * h2 + 2 * e], y[8 * h2 + 2 * e + 1]);
        }
        *reinterpret_cast<u32x4*>(zp + blk * 32 + 16 * h2) = w;
      }
    }
    if (t + stride < total) in_rows(t + stride);
  }
}

// ---------------------------------------------------------------------------------------------------------------- fp32 prologue / epilogue
constexpr int PF_R = 32, PF_CC = 16, PF_CM = 128;

__global__ void __launch_bounds__(256) triattn_prologue_f32(const float* __restrict__ z, const float* __restrict__ ln_w, const float* __restrict__ ln_b,
                                                            float eps, const float* __restrict__ w_qkvg, const float* __restrict__ w_b, int C, int H,
                                                            int D, float* __restrict__ qo, float* __restrict__ ko, float* __restrict__ vo,
                                                            float* __restrict__ go, float* __restrict__ bo, int64_t N, int ending,
                                                            const float* __restrict__ b_g) {
  __shared__ float xs[PF_R][PF_CM + 1];
  __shared__ float ws[PF_CC][PF_CM + 1];
  const int tid = threadIdx.x;
  const int64_t tpr = cdiv(N, PF_R);
  const int64_t i = blockIdx.x / tpr, j0 = (blockIdx.x % tpr) * PF_R;
  const int64_t b = blockIdx.y;
  const int HD = H * D;
  for (int c = tid; c < PF_R * C; c += 256) {
    const int r = c / C, cc = c % C;
    const int64_t j = j0 + r;
    const bool live = i < N && j < N;
    const int64_t zpix = ending ? (b * N + j) * N + i : (b * N + i) * N + j;
    xs[r][cc] = live ? z[zpix * C + cc] : 0.f;
  }
  __syncthreads();
  {
    const int r = tid >> 3, sub = tid & 7;
    float s = 0.f;
    for (int cc = sub; cc < C; cc += 8) s += xs[r][cc];
    for (int o = 4; o >= 1; o >>= 1) s += __shfl_xor(s, o, 8);
    const float mean = s / (float)C;
    float q = 0.f;
    for (int cc = sub; cc < C; cc += 8) {
      const float d = xs[r][cc] - mean;
      q += d * d;
    }
    for (int o = 4; o >= 1; o >>= 1) q += __shfl_xor(q, o, 8);
    const float rstd = 1.0f / sqrtf(q / (float)C + eps);
    __syncthreads();
    for (int cc = sub; cc < C; cc += 8) xs[r][cc] = (xs[r][cc] - mean) * rstd * (ln_w ? ln_w[cc] : 1.f) + (ln_b ? ln_b[cc] : 0.f);
  }
  const int r = tid >> 3, sub = tid & 7;
  const int64_t j = j0 + r;
  const bool live = i < N && j < N;
  const int nout = 4 * HD + H;
  for (int c0 = 0; c0 < nout; c0 += PF_CC) {
    __syncthreads();
    for (int c = tid; c < PF_CC * C; c += 256) {
      const int jj = c / C, cc = c % C, ch = c0 + jj;
      ws[jj][cc] = ch < 4 * HD ? w_qkvg[(int64_t)ch * C + cc] : (ch < nout ? w_b[(int64_t)(ch - 4 * HD) * C + cc] : 0.f);
    }
    __syncthreads();
    for (int jj = 0; jj < 2; ++jj) {
      const int oc = sub * 2 + jj, ch = c0 + oc;
      if (ch >= nout || !live) continue;
      float acc = 0.f;
      for (int cc = 0; cc < C; ++cc) acc = fmaf(xs[r][cc], ws[oc][cc], acc);
      if (ch < 3 * HD) {
        const int part = ch / HD, hd = ch % HD, hh = hd / D, d = hd % D;
        float* dst = part == 0 ? qo : (part == 1 ? ko : vo);
        dst[(((b * N + i) * H + hh) * N + j) * D + d] = acc;
      } else if (ch < 4 * HD) {
        go[((b * N + i) * N + j) * HD + (ch - 3 * HD)] = b_g ? acc + b_g[ch - 3 * HD] : acc;
      } else {
        bo[((b * H + (ch - 4 * HD)) * N + i) * N + j] = acc;
      }
    }
  }
}

__global__ void __launch_bounds__(256) triattn_epilogue_f32(const float* __restrict__ o, const float* __restrict__ gt, const float* __restrict__ w_o,
                                                            const float* __restrict__ b_o, int C, int H, int D, float* zout, int64_t N, int ending,
                                                            int residual) {
  __shared__ float xs[PF_R][PF_CM + 1];
  __shared__ float ws[PF_CC][PF_CM + 1];
  const int tid = threadIdx.x;
  const int64_t tpr = cdiv(N, PF_R);
  const int64_t i = blockIdx.x / tpr, j0 = (blockIdx.x % tpr) * PF_R;
  const int64_t b = blockIdx.y;
  const int HD = H * D;
  for (int c = tid; c < PF_R * HD; c += 256) {
    const int r = c / HD, hd = c % HD, hh = hd / D, d = hd % D;
    const int64_t j = j0 + r;
    const bool live = i < N && j < N;
    float v = 0.f;
    if (live) {
      const float gg = gt[((b * N + i) * N + j) * HD + hd];
      v = sigmoid_exact(gg) * o[(((b * N + i) * H + hh) * N + j) * D + d];
    }
    xs[r][hd] = v;
  }
  const int r = tid >> 3, sub = tid & 7;
  const int64_t j = j0 + r;
  const bool live = i < N && j < N;
  const int64_t zpix = ending ? (b * N + j) * N + i : (b * N + i) * N + j;
  for (int c0 = 0; c0 < C; c0 += PF_CC) {
    __syncthreads();
    for (int c = tid; c < PF_CC * HD; c += 256) {
      const int jj = c / HD, hd = c % HD;
      ws[jj][hd] = c0 + jj < C ? w_o[(int64_t)(c0 + jj) * HD + hd] : 0.f;
    }
    __syncthreads();
    for (int jj = 0; jj < 2; ++jj) {
      const int co = c0 + sub * 2 + jj;
      if (co >= C || !live) continue;
      float acc = 0.f;
      for (int hd = 0; hd < HD; ++hd) acc = fmaf(xs[r][hd], ws[sub * 2 + jj][hd], acc);
      if (b_o) acc += b_o[co];
      float* p = zout + zpix * C + co;
      *p = residual ? *p + acc : acc;
    }
  }
}

// dry = true: every check, nothing launched
// Sv: the real keys / queries of a block-layout call whose key axis is padded (S = Sv rounded up to 64); -1: S.  qmul > 0: a block-layout call whose q and k hold only the
// Sv real rows, q not yet multiplied by the scale -- the core multiplies q by qmul in registers and re-reads the last real key
// row for the padding keys (the op face's in-place route); 0: q and k hold S rows, q already multiplied.
static int core_launch(const FpfTriattnArgs* a, hipStream_t st, char* err, size_t errlen, bool dry = false, int64_t Sv = -1,
                       float qmul = 0.0f) {
  if (a->dtype == FPF_DT_BF16) {
    if (a->D != TA_D) return fail(err, errlen, FPF_E_SHAPE, "bf16 core serves head_dim 32 (got %lld)", (long long)a->D);
    CoreParams p{};
    p.q = (const uint16_t*)a->q;
    p.k = (const uint16_t*)a->k;
    p.v = (const uint16_t*)a->v;
    for (int t = 0; t < 5; ++t) {
      p.qs[t] = a->q_stride[t];
      p.ks[t] = a->k_stride[t];
      p.vs[t] = a->v_stride[t];
      p.os[t] = a->out_stride[t];
    }
    for (int t = 0; t < 4; ++t) p.bs[t] = a->bias_stride[t];
    for (int t = 0; t < 3; ++t) p.ms[t] = a->mask_stride[t];
    p.bias = a->bias;
    p.bias_bf16 = a->bias_dtype == FPF_DT_BF16;
    p.mask = a->mask;
    p.mask_f32 = a->mask_dtype == FPF_DT_F32;
    p.out = (uint16_t*)a->out;
    p.B = a->B;
    p.N = a->N;
    p.H = a->H;
    p.S = a->S;
    p.scale = a->scale;
    p.Sv = Sv < 0 ? a->S : Sv;
    p.qmul = qmul > 0.f ? qmul : 1.0f;
    p.Sqk = qmul > 0.f ? p.Sv : a->S;
    p.v_t = a->v_layout;
    if (!(p.v_t >= 0 && p.v_t <= 3)) return fail(err, errlen, FPF_E_ARGS, "v_layout %d", a->v_layout);
    p.v_rows = p.v_t == 3;
    for (int t = 0; t < 4; ++t)
      if ((p.qs[t] | p.ks[t] | p.vs[t]) & 7) return fail(err, errlen, FPF_E_ALIGN, "bf16 core: q / k / v strides must be multiples of 8 elements");
    for (int t = 0; t < 4; ++t)
      if (p.os[t] & 3) return fail(err, errlen, FPF_E_ALIGN, "bf16 core: out strides must be multiples of 4 elements");
    if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || (reinterpret_cast<uintptr_t>(a->out) & 7))
      return fail(err, errlen, FPF_E_ALIGN, "bf16 core: q / k / v 16-byte, out 8-byte aligned");
    p.bias_vec = !p.bias_bf16 && aligned16(a->bias) && (p.bs[0] % 4 == 0) && (p.bs[1] % 4 == 0) && (p.bs[2] % 4 == 0) && (p.S % 4 == 0);
    const int64_t total = a->B * a->H * cdiv(a->N, TA_R) * cdiv(a->S, 128);
    if (cdiv(total, 8) * 8 > 0x7fffffffLL) return fail(err, errlen, FPF_E_SHAPE, "grid too large");
    const dim3 grid((unsigned)(cdiv(total, 8) * 8)), block(256);
    if (p.v_t >= 2) {                  // the block layout (q times the scale; V^T keys permuted in 16-blocks, or V as key rows):
                                       // the DMA-staged core
      if (!p.bias_vec || p.S % TA_KT != 0 || p.S > 64 * TA_MAXW || p.vs[3] % 8 != 0)
        return fail(err, errlen, FPF_E_SHAPE, "v_layout 2 / 3 needs an fp32 16-byte-aligned bias and S a multiple of 64 up to %d", 64 * TA_MAXW);
      if (p.bs[2] != p.S || p.bs[3] != 1)
        return fail(err, errlen, FPF_E_SHAPE, "v_layout 2 / 3 reads contiguous S x S bias planes in 32 x 32 register-order blocks (bias_stride[2] = S, [3] = 1)");
      if (p.scale != 1.0f) return fail(err, errlen, FPF_E_ARGS, "v_layout 2 / 3 takes q already multiplied by the scale (scale must be 1)");
      if (!(p.qmul > 0.f) || !std::isfinite(p.qmul) || p.Sqk <= p.S - TA_KT || p.Sqk > p.S)
        return fail(err, errlen, FPF_E_ARGS, "v_layout 2 / 3: q / k rows %lld of %lld, q factor %g", (long long)p.Sqk, (long long)p.S, (double)p.qmul);
      if (p.mask && !a->keep)
        return fail(err, errlen, FPF_E_ARGS, "v_layout 2 / 3 reads the mask as a keep-bit table (keep); the fused block builds it");
      if (p.os[3] != TA_D || ((p.os[0] | p.os[1] | p.os[2]) & 7) || !aligned16(a->out))
        return fail(err, errlen, FPF_E_ALIGN, "v_layout 2 / 3 writes out rows of %d contiguous bf16, 16-byte aligned", TA_D);
      const size_t need = (size_t)redo_words(a->B, a->N, a->H, a->S) * 4;
      if (!a->workspace || a->workspace_bytes < need)
        return fail(err, errlen, FPF_E_WORKSPACE, "v_layout 2 / 3: workspace %zu < %zu bytes", (size_t)a->workspace_bytes, need);
      p.keep = a->keep;
      p.redo = static_cast<uint32_t*>(a->workspace);
      return pipe_core_launch(p, st, err, errlen, dry);
    }
    if (dry) return FPF_OK;
    if (p.v_t && p.bias_vec) hipLaunchKernelGGL((triattn_core_bf16<true, true>), grid, block, 0, st, p);
    else if (p.v_t) hipLaunchKernelGGL((triattn_core_bf16<true, false>), grid, block, 0, st, p);
    else if (p.bias_vec) hipLaunchKernelGGL((triattn_core_bf16<false, true>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((triattn_core_bf16<false, false>), grid, block, 0, st, p);
    return launched(err, errlen, "triattn_core_bf16");
  }
  if (a->dtype == FPF_DT_F32) {
    if (a->v_layout != 0) return fail(err, errlen, FPF_E_ARGS, "fp32 core takes v as [B, N, H, S, D] (v_layout 0)");
    CoreParamsF p{};
    p.q = (const float*)a->q;
    p.k = (const float*)a->k;
    p.v = (const float*)a->v;
    for (int t = 0; t < 5; ++t) {
      p.qs[t] = a->q_stride[t];
      p.ks[t] = a->k_stride[t];
      p.vs[t] = a->v_stride[t];
      p.os[t] = a->out_stride[t];
    }
    for (int t = 0; t < 4; ++t) p.bs[t] = a->bias_stride[t];
    for (int t = 0; t < 3; ++t) p.ms[t] = a->mask_stride[t];
    p.bias = a->bias;
    p.bias_bf16 = a->bias_dtype == FPF_DT_BF16;
    p.mask = a->mask;
    p.mask_f32 = a->mask_dtype == FPF_DT_F32;
    p.out = (float*)a->out;
    p.B = a->B;
    p.N = a->N;
    p.H = a->H;
    p.S = a->S;
    p.scale = a->scale;
    const int64_t blocks = a->B * a->N * a->H * cdiv(a->S, TF_QT);
    if (blocks > 0x7fffffffLL) return fail(err, errlen, FPF_E_SHAPE, "grid too large");
    if (a->D != 16 && a->D != 32 && a->D != 64) return fail(err, errlen, FPF_E_SHAPE, "fp32 core serves head_dim 16 | 32 | 64 (got %lld)", (long long)a->D);
    if (dry) return FPF_OK;
#define FPF_TF(DD)                                                                                       \
  if (a->D == DD) {                                                                                      \
    hipLaunchKernelGGL(triattn_core_f32<DD>, dim3((unsigned)blocks), dim3(TF_QT), 0, st, p);             \
    return launched(err, errlen, "triattn_core_f32");                                                    \
  }
    FPF_TF(16) FPF_TF(32) FPF_TF(64)
#undef FPF_TF
    return fail(err, errlen, FPF_E_SHAPE, "fp32 core serves head_dim 16 | 32 | 64 (got %lld)", (long long)a->D);
  }
  return fail(err, errlen, FPF_E_DTYPE, "dtype %d", a->dtype);
}

// The op face on the block-layout core: a bf16 call with head_dim 32 and S the block core serves (a multiple of 64, or at
// least 128, up to 8192), given a workspace of fpf_triattn_stage_bytes, has the bias restaged (op_stage_launch: times log2(e)
// in blocks, padded to Sp = S rounded up to 64), its mask (and the padding) becomes a keep table, and the persistent core
// reads the caller's q, k and v in place -- q multiplied by scale * log2(e) in registers, the padding keys re-reading the last
// real key row, masked -- and writes the caller's out directly.  V given transposed (v_layout 1) is restaged as V^T in the
// core's key order.  Workspace regions: v2 (B N H 32 Sp bf16, V^T only) | bias2 (B H Sp^2 fp32) | keep | redo.
struct OpStage {
  size_t bias2, keep, redo, total;
};
static OpStage op_stage_layout(int64_t B, int64_t N, int64_t H, int64_t S) {
  const int64_t Sp = block_np(FPF_DT_BF16, S);
  const auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
  const size_t r = al((size_t)B * N * H * Sp * TA_D * 2), rb = al((size_t)B * H * Sp * Sp * 4);
  const size_t rk = al((size_t)B * N * keep_words(Sp) * 8), rr = al((size_t)redo_words(B, N, H, Sp) * 4);
  return {r, r + rb, r + rb + rk, r + rb + rk + rr};
}
static bool op_staged_shape(int dtype, int64_t D, int64_t S) { return dtype == FPF_DT_BF16 && D == TA_D && block_layout2(dtype, S); }
static bool rows32_ok(const void* p, const int64_t* st4) {     // rows of 32 contiguous bf16, 16-byte aligned, for strides [0..3]
  return aligned16(p) && ((st4[0] | st4[1] | st4[2] | st4[3]) & 7) == 0;
}

// the caller's q, k and v strides (or, for V^T given transposed, the staged copy's) within the block-layout core's 32-bit
// in-item offsets
static bool op_in_place_fits(const FpfTriattnArgs* a) {
  const int64_t Sp = block_np(FPF_DT_BF16, a->S);
  if (a->v_layout == 0) return pipe_offsets_fit(Sp, a->q_stride, a->k_stride, a->v_stride, true);
  const int64_t vs5[5] = {a->N * a->H * TA_D * Sp, a->H * TA_D * Sp, TA_D * Sp, Sp, 1};
  return pipe_offsets_fit(Sp, a->q_stride, a->k_stride, vs5, false);
}

static int op_staged(const FpfTriattnArgs* a, hipStream_t st, char* err, size_t errlen) {
  const int64_t B = a->B, N = a->N, H = a->H, S = a->S, Sp = block_np(FPF_DT_BF16, S);
  const OpStage L = op_stage_layout(B, N, H, S);
  char* w = static_cast<char*>(a->workspace);
  const bool v_rows = a->v_layout == 0;            // V as key rows, read in place (V^T: restaged)
  StageParams sp{};
  sp.v = (const uint16_t*)a->v;
  for (int t = 0; t < 4; ++t) sp.vs[t] = a->v_stride[t];
  sp.v_t = a->v_layout;
  sp.bias = a->bias;
  sp.bias_bf16 = a->bias_dtype == FPF_DT_BF16;
  for (int t = 0; t < 3; ++t) sp.bs[t] = a->bias_stride[t];
  sp.v2 = v_rows ? nullptr : reinterpret_cast<uint16_t*>(w);
  sp.bias2 = reinterpret_cast<float*>(w + L.bias2);
  sp.B = B;
  sp.N = N;
  sp.H = H;
  sp.S = S;
  sp.Sp = Sp;
  uint64_t* keep = reinterpret_cast<uint64_t*>(w + L.keep);
  FpfTriattnArgs c = *a;
  c.v_layout = v_rows ? 3 : 2;
  c.S = Sp;
  if (!v_rows) {
    const int64_t vs5[5] = {N * H * TA_D * Sp, H * TA_D * Sp, TA_D * Sp, Sp, 1};
    for (int t = 0; t < 5; ++t) c.v_stride[t] = vs5[t];
    c.v = sp.v2;
  }
  c.bias = sp.bias2;
  c.bias_dtype = FPF_DT_F32;
  c.bias_stride[0] = H * Sp * Sp;
  c.bias_stride[1] = Sp * Sp;
  c.bias_stride[2] = Sp;
  c.bias_stride[3] = 1;
  c.scale = 1.0f;
  c.keep = (a->mask || Sp != S) ? keep : nullptr;
  c.workspace = w + L.redo;
  c.workspace_bytes = L.total - L.redo;
  for (int pass = 0; pass < 2; ++pass) {            // every check of every stage before the first launch
    const bool dry = pass == 0;
    int rc = op_stage_launch(sp, st, err, errlen, dry);
    if (rc) return rc;
    if (c.keep) {
      rc = keep_table_launch(a->mask, a->mask_dtype == FPF_DT_F32, a->mask_stride, B, N, Sp, S, keep, st, err, errlen, dry);
      if (rc) return rc;
    }
    rc = core_launch(&c, st, err, errlen, dry, S, a->scale * LOG2E);
    if (rc || !dry) return rc;
  }
  return FPF_OK;
}

}  // namespace fpf

extern "C" size_t fpf_triattn_stage_bytes(int64_t B, int64_t N, int64_t H, int64_t S, int64_t D, int32_t dtype) {
  using namespace fpf;
  if (B <= 0 || N <= 0 || H <= 0 || !op_staged_shape(dtype, D, S)) return 0;
  return op_stage_layout(B, N, H, S).total;
}

extern "C" int fpf_triattn_fwd(const FpfTriattnArgs* a, void* stream, char* err, size_t errlen) {
  using namespace fpf;
  FPF_CHECK_VERSION(a);
  if (!a->q || !a->k || !a->v || !a->bias || !a->out) return fail(err, errlen, FPF_E_ARGS, "q / k / v / bias / out is NULL");
  if (a->B < 0 || a->N < 0 || a->H <= 0 || a->S < 0 || a->D <= 0) return fail(err, errlen, FPF_E_SHAPE, "negative extent");
  if (a->B == 0 || a->N == 0 || a->S == 0) return FPF_OK;
  if (a->q_stride[4] != 1 || a->k_stride[4] != 1 || a->v_stride[4] != 1 || a->out_stride[4] != 1 || a->bias_stride[3] != 1)
    return fail(err, errlen, FPF_E_SHAPE, "the last (head_dim / key) strides must be 1");
  if (!(a->bias_dtype == FPF_DT_F32 || a->bias_dtype == FPF_DT_BF16)) return fail(err, errlen, FPF_E_DTYPE, "bias_dtype %d", a->bias_dtype);
  if (a->mask && !(a->mask_dtype == FPF_DT_U8 || a->mask_dtype == FPF_DT_F32)) return fail(err, errlen, FPF_E_DTYPE, "mask_dtype %d", a->mask_dtype);
  if (!(a->scale > 0.f)) return fail(err, errlen, FPF_E_ARGS, "scale must be > 0");
  if ((a->v_layout == 0 || a->v_layout == 1) && a->workspace && op_staged_shape(a->dtype, a->D, a->S) &&
      a->workspace_bytes >= op_stage_layout(a->B, a->N, a->H, a->S).total && rows32_ok(a->q, a->q_stride) &&
      rows32_ok(a->k, a->k_stride) && rows32_ok(a->v, a->v_stride) && aligned16(a->out) && a->out_stride[3] == TA_D &&
      ((a->out_stride[0] | a->out_stride[1] | a->out_stride[2]) & 7) == 0 &&
      op_in_place_fits(a))
    return op_staged(a, static_cast<hipStream_t>(stream), err, errlen);
  return core_launch(a, static_cast<hipStream_t>(stream), err, errlen);
}

extern "C" size_t fpf_triattn_workspace_bytes(int64_t B, int64_t N, int64_t H, int64_t S, int32_t v_layout) {
  if ((v_layout != 2 && v_layout != 3) || B <= 0 || N <= 0 || H <= 0 || S <= 0) return 0;
  return (size_t)fpf::redo_words(B, N, H, S) * 4;
}

namespace fpf {

// Shape / alignment gate shared by the block and its two stages.
static int block_shape_check(int dtype, int64_t B, int C, int64_t H, int64_t D, char* err, size_t errlen) {
  if (B > 65535) return fail(err, errlen, FPF_E_SHAPE, "B above 65535");
  if (dtype == FPF_DT_BF16) {
    if (C != TP_C || H * D != TP_HD || D != TA_D) return fail(err, errlen, FPF_E_SHAPE, "bf16 block serves C = 128, H*D = 128, D = 32");
    return FPF_OK;
  }
  if (dtype == FPF_DT_F32) {
    if (C > PF_CM || H * D > PF_CM || C <= 0 || H <= 0 || D <= 0) return fail(err, errlen, FPF_E_SHAPE, "fp32 block serves C, H*D <= 128");
    return FPF_OK;
  }
  return fail(err, errlen, FPF_E_DTYPE, "dtype %d", dtype);
}

// The bf16 block with N a multiple of 64 (up to 8192) runs the block-layout core (v_layout 2): its q carries scale * log2(e),
// its bias (computed in the block or by fpf_triattn_bias_fwd for bias_in) log2(e).


static int prologue_launch(int dtype, const void* z, const float* ln_w, const float* ln_b, float eps, const void* w_qkvg, const void* w_b,
                           int64_t B, int64_t N, int C, int H, int D, int ending, void* q, void* k, void* v, int64_t v_ld, void* g, float* bias,
                           hipStream_t st, char* err, size_t errlen, int flags = PRO_QKV | PRO_G | PRO_BIAS, int64_t row0 = 0,
                           int64_t rows = -1, float q_scale = 1.0f, float bias_scale = 1.0f, int64_t bias_ld = -1, int bias_bf16 = 0,
                           const float* b_g = nullptr, bool dry = false, int64_t Np = -1, const void* xln = nullptr) {
  if (rows < 0) rows = N;
  if (bias_ld < 0) bias_ld = N;
  if (Np < 0) Np = N;
  if (Np != N && (dtype != FPF_DT_BF16 || !(flags & PRO_BIAS_BLK) || (flags & PRO_G) || Np % 64 || Np < N))
    return fail(err, errlen, FPF_E_SHAPE, "a padded J extent (%lld for N = %lld) serves the bf16 block layout only", (long long)Np, (long long)N);
  if (dtype == FPF_DT_BF16) {
    if (!aligned16(z) || !aligned16(w_qkvg) || !aligned16(w_b) || ((flags & PRO_QKV) && (!aligned16(q) || !aligned16(k) || !aligned16(v))) ||
        ((flags & PRO_G) && !aligned16(g)) || ((flags & PRO_BIAS) && !aligned16(bias)))
      return fail(err, errlen, FPF_E_ALIGN, "prologue operands must be 16-byte aligned");
    if ((flags & PRO_QKV) && (v_ld < cdiv(Np, 32) * 32 || v_ld % 8))
      return fail(err, errlen, FPF_E_SHAPE, "v_ld %lld: V^T rows need %lld rounded up to 32", (long long)v_ld, (long long)Np);
    if ((flags & PRO_BIAS_BLK) && (Np % 32 || bias_ld != N || bias_bf16))
      return fail(err, errlen, FPF_E_SHAPE, "blocked bias: fp32, a J extent that is a multiple of 32, contiguous planes");
    ProParams p{};
    p.z = (const uint16_t*)z;
    p.ln_w = ln_w;
    p.ln_b = ln_b;
    p.eps = eps;
    p.w_qkvg = (const uint16_t*)w_qkvg;
    p.w_b = (const uint16_t*)w_b;
    p.H = H;
    p.q = (uint16_t*)q;
    p.k = (uint16_t*)k;
    p.v = (uint16_t*)v;
    p.g = (uint16_t*)g;
    p.bias = bias;
    p.N = N;
    p.Jp = v_ld;
    p.Np = Np;
    p.B = B;
    p.row0 = row0;
    p.rows = rows;
    p.ending = ending;
    p.flags = flags;
    p.q_scale = q_scale;
    p.bias_scale = bias_scale;
    p.bias_ld = bias_ld;
    p.bias_bf16 = bias_bf16;
    p.b_g = b_g;
    if (!rt_tiles_ok(B * rows * cdiv(Np, 32))) return fail(err, errlen, FPF_E_SHAPE, "prologue: 2^31 or more 32-pixel tiles");
    if (xln && !aligned16(xln)) return fail(err, errlen, FPF_E_ALIGN, "x_ln must be 16-byte aligned");
    p.xln = static_cast<const uint16_t*>(xln);
    if (dry) return FPF_OK;
    const unsigned grid = (unsigned)std::min<int64_t>(num_cus(), cdiv(B * rows * cdiv(Np, 32), RT_WAVES));
    if (xln) hipLaunchKernelGGL(triattn_prologue_bf16<true>, dim3(grid), dim3(512), 0, st, p);
    else hipLaunchKernelGGL(triattn_prologue_bf16<false>, dim3(grid), dim3(512), 0, st, p);
    return launched(err, errlen, "triattn_prologue_bf16");
  }
  if (row0 != 0 || rows != N || flags != (PRO_QKV | PRO_G | PRO_BIAS) || q_scale != 1.0f || bias_scale != 1.0f || bias_ld != N || bias_bf16)
    return fail(err, errlen, FPF_E_SHAPE, "the fp32 prologue serves whole tensors (no row range, every output, q unscaled)");
  if (xln) return fail(err, errlen, FPF_E_DTYPE, "x_ln serves the bf16 prologue");
  if (dry) return FPF_OK;
  const unsigned grid = (unsigned)(N * cdiv(N, PF_R));
  hipLaunchKernelGGL(triattn_prologue_f32, dim3(grid, (unsigned)B), dim3(256), 0, st, (const float*)z, ln_w, ln_b, eps, (const float*)w_qkvg,
                     (const float*)w_b, C, H, D, (float*)q, (float*)k, (float*)v, (float*)g, bias, N, ending, b_g);
  return launched(err, errlen, "triattn_prologue_f32");
}

static int epilogue_launch(int dtype, const void* o, const void* g, const void* w_o, const float* b_o, int64_t B, int64_t N, int C, int H,
                           int D, int ending, int residual, void* out, hipStream_t st, char* err, size_t errlen, bool dry = false) {
  if (dtype == FPF_DT_BF16) {
    if (!aligned16(o) || !aligned16(g) || !aligned16(w_o) || !aligned16(out))
      return fail(err, errlen, FPF_E_ALIGN, "epilogue operands must be 16-byte aligned");
    if (!rt_tiles_ok(B * N * cdiv(N, 32))) return fail(err, errlen, FPF_E_SHAPE, "epilogue: 2^31 or more 32-pixel tiles");
    if (dry) return FPF_OK;
    const unsigned grid = (unsigned)std::min<int64_t>(2 * num_cus(), cdiv(B * N * cdiv(N, 32), RT_WAVES));
    hipLaunchKernelGGL(triattn_epilogue_bf16, dim3(grid), dim3(512), 0, st, (const uint16_t*)o, (const uint16_t*)g, (const uint16_t*)w_o, b_o,
                       H, (uint16_t*)out, N, B, ending, residual);
    return launched(err, errlen, "triattn_epilogue_bf16");
  }
  if (dry) return FPF_OK;
  const unsigned grid = (unsigned)(N * cdiv(N, PF_R));
  hipLaunchKernelGGL(triattn_epilogue_f32, dim3(grid, (unsigned)B), dim3(256), 0, st, (const float*)o, (const float*)g, (const float*)w_o, b_o, C,
                     H, D, (float*)out, N, ending, residual);
  return launched(err, errlen, "triattn_epilogue_f32");
}

}  // namespace fpf

extern "C" int fpf_triattn_prologue_fwd(const FpfTriattnPrologueArgs* a, void* stream, char* err, size_t errlen) {
  using namespace fpf;
  FPF_CHECK_VERSION(a);
  if (!a->z || !a->w_qkvg || !a->w_b || !a->q || !a->k || !a->v || !a->g || !a->bias)
    return fail(err, errlen, FPF_E_ARGS, "z / weights / q / k / v / g / bias is NULL");
  if (a->B < 0 || a->N < 0) return fail(err, errlen, FPF_E_SHAPE, "negative extent");
  if (a->B == 0 || a->N == 0) return FPF_OK;
  const int rc = block_shape_check(a->dtype, a->B, a->C, a->H, a->D, err, errlen);
  if (rc) return rc;
  return prologue_launch(a->dtype, a->z, a->ln_w, a->ln_b, a->eps, a->w_qkvg, a->w_b, a->B, a->N, a->C, a->H, a->D, a->ending, a->q, a->k, a->v,
                         a->v_ld, a->g, a->bias, static_cast<hipStream_t>(stream), err, errlen, PRO_QKV | PRO_G | PRO_BIAS, 0, -1, 1.0f, 1.0f, -1, 0,
                         a->b_g, false, -1, a->x_ln);
}

extern "C" int fpf_triattn_epilogue_fwd(const FpfTriattnEpilogueArgs* a, void* stream, char* err, size_t errlen) {
  using namespace fpf;
  FPF_CHECK_VERSION(a);
  if (!a->o || !a->g || !a->w_o || !a->out) return fail(err, errlen, FPF_E_ARGS, "o / g / w_o / out is NULL");
  if (a->B < 0 || a->N < 0) return fail(err, errlen, FPF_E_SHAPE, "negative extent");
  if (a->B == 0 || a->N == 0) return FPF_OK;
  const int rc = block_shape_check(a->dtype, a->B, a->C, a->H, a->D, err, errlen);
  if (rc) return rc;
  return epilogue_launch(a->dtype, a->o, a->g, a->w_o, a->b_o, a->B, a->N, a->C, a->H, a->D, a->ending, a->residual, a->out,
                         static_cast<hipStream_t>(stream), err, errlen);
}

extern "C" size_t fpf_triattn_block_workspace_bytes(int64_t B, int64_t N, int64_t rows, int32_t C, int32_t H, int32_t D, int32_t dtype) {
  (void)C;
  if (rows <= 0 || rows > N) rows = N;
  const size_t elt = dtype == FPF_DT_F32 ? 4 : 2;
  const int64_t Np = fpf::block_np(dtype, N), Jp = fpf::block_layout2(dtype, N) ? Np : fpf::cdiv(N, 32) * 32;
  const size_t HD = (size_t)H * (size_t)D;
  // q, k, v, o (and g for fp32: the bf16 epilogue recomputes the gate) of `rows` attention rows (HD per position each, Jp
  // positions: N rounded up to 64 for the block-layout core, to 32 otherwise) + the full bias (H fp32 planes of Np x Np),
  // 256-byte aligned regions
  const size_t r1 = ((size_t)B * rows * Jp * HD * elt + 255) & ~(size_t)255;
  const size_t r2 = ((size_t)B * (size_t)Np * (size_t)Np * (size_t)H * 4 + 255) & ~(size_t)255;
  // + the keep-bit table of the block-layout core (B x rows attention rows, Np / 64 + 1 words each) and its redo flags
  const size_t r3 = ((size_t)B * rows * (size_t)fpf::keep_words(Np) * 8 + 255) & ~(size_t)255;
  const size_t r4 = ((size_t)fpf::redo_words(B, rows, H, Np) * 4 + 255) & ~(size_t)255;
  return (dtype == FPF_DT_F32 ? 5 : 4) * r1 + r2 + r3 + r4;
}

extern "C" size_t fpf_triattn_bias_bytes(int64_t B, int64_t N, int32_t H, int32_t dtype) {
  if (B <= 0 || N <= 0 || H <= 0) return 0;
  const int64_t Np = fpf::block_np(dtype, N);
  return (size_t)B * (size_t)H * (size_t)Np * (size_t)Np * 4;
}

extern "C" int fpf_triattn_bias_fwd(const FpfTriattnBiasArgs* a, void* stream, char* err, size_t errlen) {
  using namespace fpf;
  FPF_CHECK_VERSION(a);
  if (!a->z || !a->w_b || !a->bias) return fail(err, errlen, FPF_E_ARGS, "z / w_b / bias is NULL");
  if (a->B <= 0 || a->N <= 0) return a->B == 0 || a->N == 0 ? FPF_OK : fail(err, errlen, FPF_E_SHAPE, "negative extent");
  if (a->dtype != FPF_DT_BF16) return fail(err, errlen, FPF_E_DTYPE, "the bias pass serves the bf16 block");
  const int rc = block_shape_check(a->dtype, a->B, a->C, a->H, a->D, err, errlen);
  if (rc) return rc;
  // the prologue kernel with only its bias output (the q|k|v|g weights are neither staged nor read)
  return prologue_launch(a->dtype, a->z, a->ln_w, a->ln_b, a->eps, a->w_qkvg ? a->w_qkvg : a->w_b, a->w_b, a->B, a->N, a->C, a->H, a->D, a->ending,
                         nullptr, nullptr, nullptr, 0, nullptr, a->bias, static_cast<hipStream_t>(stream), err, errlen,
                         PRO_BIAS | (block_layout2(a->dtype, a->N) ? PRO_BIAS_BLK : 0), 0, -1, 1.0f, block_layout2(a->dtype, a->N) ? LOG2E : 1.0f, -1, 0,
                         nullptr, false, block_np(a->dtype, a->N));
}

extern "C" int fpf_apb_bias_fwd(const FpfApbBiasArgs* a, void* stream, char* err, size_t errlen) {
  using namespace fpf;
  FPF_CHECK_VERSION(a);
  if (!a->z || !a->w_z || !a->bias) return fail(err, errlen, FPF_E_ARGS, "z / w_z / bias is NULL");
  if (a->B < 0 || a->N < 0) return fail(err, errlen, FPF_E_SHAPE, "negative extent");
  if (a->B == 0 || a->N == 0) return FPF_OK;
  if (a->dtype != FPF_DT_BF16) return fail(err, errlen, FPF_E_DTYPE, "the pair-bias producer reads bf16 z");
  if (a->C != TP_C || a->H < 1 || a->H > 32) return fail(err, errlen, FPF_E_SHAPE, "the pair-bias producer serves C = 128, 1 <= H <= 32 (got C=%d H=%d)", a->C, a->H);
  if (a->B > 65535) return fail(err, errlen, FPF_E_SHAPE, "B above 65535");
  if (!(a->bias_dtype == FPF_DT_F32 || a->bias_dtype == FPF_DT_BF16)) return fail(err, errlen, FPF_E_DTYPE, "bias_dtype %d", a->bias_dtype);
  const int64_t ld = a->bias_ld > 0 ? a->bias_ld : a->N;
  if (ld < a->N) return fail(err, errlen, FPF_E_SHAPE, "bias_ld %lld < N %lld", (long long)ld, (long long)a->N);
  return prologue_launch(a->dtype, a->z, a->ln_w, a->ln_b, a->eps, a->w_z, a->w_z, a->B, a->N, a->C, a->H, 1, 0, nullptr, nullptr, nullptr, 0,
                         nullptr, static_cast<float*>(a->bias), static_cast<hipStream_t>(stream), err, errlen, PRO_BIAS, 0, -1, 1.0f, 1.0f, ld,
                         a->bias_dtype == FPF_DT_BF16);
}

extern "C" int fpf_triattn_block_fwd(const FpfTriattnBlockArgs* a, void* stream, char* err, size_t errlen) {
  using namespace fpf;
  FPF_CHECK_VERSION(a);
  if (!a->z || !a->w_qkvg || !a->w_b || !a->w_o || !a->out) return fail(err, errlen, FPF_E_ARGS, "z / weights / out is NULL");
  if (a->B <= 0 || a->N <= 0) return a->B == 0 || a->N == 0 ? FPF_OK : fail(err, errlen, FPF_E_SHAPE, "negative extent");
  if (a->residual && a->out != a->z) return fail(err, errlen, FPF_E_ARGS, "residual form updates z in place: out must be z");
  if (a->mask && !(a->mask_dtype == FPF_DT_U8 || a->mask_dtype == FPF_DT_F32)) return fail(err, errlen, FPF_E_DTYPE, "mask_dtype %d", a->mask_dtype);
  if (a->mask_frame != 0 && a->mask_frame != 1) return fail(err, errlen, FPF_E_ARGS, "mask_frame %d (0: z frame, 1: attention frame)", a->mask_frame);
  const int64_t B = a->B, N = a->N, H = a->H, D = a->D, HD = H * D;
  const int64_t R = a->rows > 0 ? a->rows : N, row0 = a->row0;
  if (row0 < 0 || row0 + R > N) return fail(err, errlen, FPF_E_SHAPE, "rows [%lld, %lld) outside [0, %lld)", (long long)row0, (long long)(row0 + R), (long long)N);
  const bool ranged = R < N;
  if (ranged && a->dtype != FPF_DT_BF16) return fail(err, errlen, FPF_E_SHAPE, "the fp32 block serves whole tensors (no row range)");
  if (ranged && !a->bias_in) return fail(err, errlen, FPF_E_ARGS, "a row range needs bias_in (the full bias from fpf_triattn_bias_fwd)");
  if (a->bias_in && a->dtype != FPF_DT_BF16) return fail(err, errlen, FPF_E_DTYPE, "bias_in serves the bf16 block");
  if (a->x_ln && (a->dtype != FPF_DT_BF16 || ranged || a->bias_in))
    return fail(err, errlen, FPF_E_ARGS, "x_ln serves the whole bf16 block (no row range, no bias_in: the bias comes from x_ln)");
  if (a->x_ln && !aligned16(a->x_ln)) return fail(err, errlen, FPF_E_ALIGN, "x_ln must be 16-byte aligned");
  const size_t need = fpf_triattn_block_workspace_bytes(B, N, R, a->C, a->H, a->D, a->dtype);
  if (!a->workspace || a->workspace_bytes < need) return fail(err, errlen, FPF_E_WORKSPACE, "workspace %zu < %zu bytes", (size_t)a->workspace_bytes, need);
  {
    const int rc = block_shape_check(a->dtype, a->B, a->C, a->H, a->D, err, errlen);
    if (rc) return rc;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t elt = a->dtype == FPF_DT_F32 ? 4 : 2;
  // bf16 up to N = 8192: the block-layout core, fed q times scale * log2(e), the bias times log2(e) and V^T keys in its
  // 16-block order, on a J axis of Np = N rounded up to 64 (the padding keys masked, the padding queries not stored)
  const bool dma_core = block_layout2(a->dtype, N);
  const int64_t Np = block_np(a->dtype, N), Jp = dma_core ? Np : cdiv(N, 32) * 32;
  const size_t r1 = ((size_t)B * R * Jp * HD * elt + 255) & ~(size_t)255;
  char* w = static_cast<char*>(a->workspace);
  const int regions = a->dtype == FPF_DT_F32 ? 5 : 4;  // q, k, v, o (+ g on the fp32 path)
  void *q = w, *k = w + r1, *v = w + 2 * r1, *o = w + 3 * r1, *g = regions == 5 ? w + 4 * r1 : nullptr;
  float* bias = a->bias_in ? const_cast<float*>(a->bias_in) : reinterpret_cast<float*>(w + regions * r1);
  uint64_t* keep = reinterpret_cast<uint64_t*>(w + regions * r1 + (((size_t)B * Np * Np * H * 4 + 255) & ~(size_t)255));
  void* redo = reinterpret_cast<char*>(keep) + (((size_t)B * R * (size_t)keep_words(Np) * 8 + 255) & ~(size_t)255);
  const float scale = a->scale > 0.f ? a->scale : 1.0f / sqrtf((float)D);
  FpfTriattnArgs c{};
  c.abi_version = FPF_ABI_VERSION;
  c.dtype = a->dtype;
  c.B = B;
  c.N = R;                                       // the attention rows of this call
  c.H = H;
  c.S = Np;
  c.D = D;
  c.q = q;
  c.k = k;
  c.v = v;
  const int64_t st5[5] = {R * H * Np * D, H * Np * D, Np * D, D, 1};
  for (int t = 0; t < 5; ++t) c.q_stride[t] = c.k_stride[t] = c.v_stride[t] = c.out_stride[t] = st5[t];
  if (a->dtype == FPF_DT_BF16) {               // the bf16 prologue writes V transposed: [B, R, H, D, Jp]
    c.v_layout = dma_core ? 2 : 1;
    c.v_stride[0] = R * H * D * Jp;
    c.v_stride[1] = H * D * Jp;
    c.v_stride[2] = D * Jp;
    c.v_stride[3] = Jp;
    c.v_stride[4] = 1;
  }
  c.bias = bias;
  c.bias_dtype = FPF_DT_F32;
  c.bias_stride[0] = H * Np * Np;
  c.bias_stride[1] = Np * Np;
  c.bias_stride[2] = Np;
  c.bias_stride[3] = 1;
  // key mask of attention row i: z-frame pair mask row i (starting) / column i (ending), rows from row0
  c.mask_dtype = a->mask_dtype;
  c.mask_stride[0] = N * N;
  const bool by_col = a->ending && !a->mask_frame;
  c.mask_stride[1] = by_col ? 1 : N;
  c.mask_stride[2] = by_col ? N : 1;
  c.mask = a->mask ? static_cast<const char*>(a->mask) + row0 * c.mask_stride[1] * (a->mask_dtype == FPF_DT_F32 ? 4 : 1) : nullptr;
  c.out = o;
  c.scale = dma_core ? 1.0f : scale;
  c.workspace = redo;
  c.workspace_bytes = (size_t)redo_words(B, R, H, Np) * 4;
  if (dma_core && (c.mask || Np != N)) c.keep = keep;   // the block-layout core reads the mask (and the padding) as keep bits
  const bool fused_gate = a->dtype == FPF_DT_BF16;      // bf16: g is recomputed in the epilogue instead of stored
  const int flags = PRO_QKV | (fused_gate ? 0 : PRO_G) | (a->bias_in ? 0 : PRO_BIAS) | (dma_core ? PRO_VPERM | PRO_BIAS_BLK : 0);
  // two passes over the stages: the first runs every check and launches nothing, so a refusal leaves the stream untouched
  for (int pass = 0; pass < 2; ++pass) {
    const bool dry = pass == 0;
    if (c.keep) {
      const int rc = keep_table_launch(c.mask, c.mask_dtype == FPF_DT_F32, c.mask_stride, B, R, Np, N, keep, st, err, errlen, dry);
      if (rc) return rc;
    }
    int rc = prologue_launch(a->dtype, a->z, a->ln_w, a->ln_b, a->eps, a->w_qkvg, a->w_b, B, N, a->C, (int)H, (int)D, a->ending, q, k, v, Jp,
                             g, bias, st, err, errlen, flags, row0, R, dma_core ? scale * LOG2E : 1.0f, dma_core ? LOG2E : 1.0f, -1, 0, a->b_g, dry,
                             Np, a->x_ln);
    if (rc) return rc;
    rc = core_launch(&c, st, err, errlen, dry, N);
    if (rc) return rc;
    if (fused_gate) {
      if (!aligned16(a->out)) return fail(err, errlen, FPF_E_ALIGN, "out must be 16-byte aligned");
      if (!rt_tiles_ok(B * R * cdiv(N, 32))) return fail(err, errlen, FPF_E_SHAPE, "epilogue: 2^31 or more 32-pixel tiles");
    } else {
      rc = epilogue_launch(a->dtype, o, g, a->w_o, a->b_o, B, N, a->C, (int)H, (int)D, a->ending, a->residual, a->out, st, err, errlen, dry);
      if (rc || !dry) return rc;
    }
  }
  {
    const unsigned grid = (unsigned)std::min<int64_t>(2 * num_cus(), cdiv(B * R * cdiv(N, 32), RT_WAVES));
    if (a->x_ln)
      hipLaunchKernelGGL(triattn_epilogue_gate_bf16<true>, dim3(grid), dim3(512), 0, st, (const uint16_t*)a->z, (const uint16_t*)o, a->ln_w,
                         a->ln_b, a->eps, (const uint16_t*)a->w_qkvg + 3 * HD * a->C, (const uint16_t*)a->w_o, a->b_g, a->b_o, (uint16_t*)a->out, N,
                         B, row0, R, a->ending, a->residual, Np, (const uint16_t*)a->x_ln);
    else
      hipLaunchKernelGGL(triattn_epilogue_gate_bf16<false>, dim3(grid), dim3(512), 0, st, (const uint16_t*)a->z, (const uint16_t*)o, a->ln_w,
                         a->ln_b, a->eps, (const uint16_t*)a->w_qkvg + 3 * HD * a->C, (const uint16_t*)a->w_o, a->b_g, a->b_o, (uint16_t*)a->out, N,
                         B, row0, R, a->ending, a->residual, Np, nullptr);
    return launched(err, errlen, "triattn_epilogue_gate_bf16");
  }
}
