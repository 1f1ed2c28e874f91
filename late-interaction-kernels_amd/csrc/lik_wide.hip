// MaxSim for embedding dims beyond the tile kernel's column blocks (bf16 /
// fp16 rows wider than 512 elements, fp32 rows wider than 256).
//
// The tile kernel holds a query block's MFMA B fragments in VGPRs for its
// whole life, which caps the row width. This kernel trades speed for reach:
// one wavefront per (query, doc) pair, both operands loaded from memory per
// 16-element k-step (the query block and the doc tile stay in L1 / L2), so
// any width works. It is the correctness path for those shapes, not a fast
// one. Same semantics as the tile kernel (reference.py:26-98): per query
// token the max over valid doc tokens of <q, t> (both L2-normalised when
// asked), a max over no token or a non-finite max counting 0, summed over
// the valid query tokens. fp32 inputs use the three-term bf16 split
// (hi*hi + hi*lo + lo*hi), as the tile kernel does.
#include "lik_kernel.h"

namespace lik {

template <int EK>
__global__ void __launch_bounds__(256) maxsim_wide_kernel(const Params p) {
  constexpr int EB = EK == EK_F32 ? 4 : 2;
  constexpr float NEG_INF = -__builtin_huge_valf();
  __shared__ __attribute__((aligned(16))) float s_sc[4][32];

  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
  const int wl = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t w = (int64_t)blockIdx.x * 4 + wl;
  // cross product / KD: wave w is (query q, doc jl); pair list: wave w is pair w
  int64_t q, jl, j;
  if (p.pair_q) {
    if (w >= p.nunits) return;  // wave-uniform; no barrier in this kernel
    q = p.pair_q[w];
    j = p.pair_d[w];
    jl = 0;
    if (q < 0 || q >= p.q.n || j < 0 || j >= p.d.n) {  // out-of-range pair: score 0, argmax stays -1
      if (lane == 0) p.out[w * p.osq] = 0.f;
      return;
    }
  } else {
    q = w / p.ndocs_pg;
    jl = w - q * p.ndocs_pg;
    if (q >= p.q.n) return;
    j = p.kd_K ? q * p.kd_K + jl : jl;
  }
  // argmax row of this (query, doc): (q * docs + jl), or the pair index
  int32_t* const arow = p.amax ? p.amax + (p.pair_q ? w : q * p.amax_qs + jl) * p.amax_ld : nullptr;
  const int64_t lq = seq_len(p.q, q), ld = seq_len(p.d, j);
  const char* q0 = seq_row0(p.q, q);
  const char* d0 = seq_row0(p.d, j);
  const int dim = p.q.dim;
  const int nk = (dim + 15) / 16;
  const bool norm_q = (p.normalize & 1) != 0, norm_d = (p.normalize & 2) != 0;

  // this lane's 8 elements [e0, e0 + 8) of row `row` (zero past the row or dim)
  auto frag = [&](const char* base, bool ok, int e0, float* v) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = 0.f;
    if (!ok || e0 >= dim) return;
    const char* ptr = base + (int64_t)e0 * EB;
    if constexpr (EK == EK_F32) {
      const f32x4 a = *(const f32x4*)ptr;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = a[e];
      if (e0 + 4 < dim) {
        const f32x4 b = *(const f32x4*)(ptr + 16);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 + e] = b[e];
      }
    } else {
      const u32x4 a = *(const u32x4*)ptr;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t wd = a[e >> 1];
        v[e] = EK == EK_BF16 ? ((e & 1) ? bf16hi_to_f32(wd) : bf16lo_to_f32(wd))
                             : f16_to_f32((uint16_t)((e & 1) ? (wd >> 16) : (wd & 0xffffu)));
      }
    }
  };
  // fp32 -> MFMA operand words: exact for 16-bit inputs, hi / lo bf16 halves for fp32
  auto pack = [&](const float* v, u32x4& hi, u32x4& lo) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (EK == EK_F16) {
        hi[k] = f32_to_f16_bits(v[2 * k]) | (f32_to_f16_bits(v[2 * k + 1]) << 16);
      } else {
        if constexpr (EK == EK_F32) {
          const uint32_t a = split_hi(v[2 * k]), b = split_hi(v[2 * k + 1]);
          hi[k] = a | (b << 16);
          lo[k] = split_lo(a, v[2 * k]) | (split_lo(b, v[2 * k + 1]) << 16);
        } else {
          hi[k] = f32_to_bf16_bits(v[2 * k]) | (f32_to_bf16_bits(v[2 * k + 1]) << 16);
        }
      }
    }
  };
  constexpr int MK = EK == EK_F16 ? EK_F16 : EK_BF16;

  float total = 0.f;
  for (int64_t qb = 0; qb < lq; qb += 32) {
    const int64_t qt = qb + l32;
    bool qv = qt < lq;
    if (qv && p.q.mask) qv = p.q.mask[q * p.q.msn + qt * p.q.msl] != 0;
    const char* qrow = q0 + qt * p.q.sl_b;
    float m = NEG_INF, ssq = 0.f;
    int mi = -1;  // doc row of m (rows visited in increasing order: first index of the max)
    for (int64_t t0 = 0; t0 < ld; t0 += 32) {
      const int64_t r = t0 + l32;
      bool rv = r < ld;
      if (rv && p.d.mask) rv = p.d.mask[j * p.d.msn + r * p.d.msl] != 0;
      const char* drow = d0 + r * p.d.sl_b;
      f32x16 acc = {};
      float ssd = 0.f;
      for (int k = 0; k < nk; ++k) {
        const int e0 = k * 16 + 8 * h;
        float a[8], b[8];
        frag(drow, r < ld, e0, a);
        frag(qrow, qt < lq, e0, b);
        u32x4 ah, al, bh, bl;
        pack(a, ah, al);
        pack(b, bh, bl);
        acc = mfma32<MK>(acc, &ah, &bh);
        if constexpr (EK == EK_F32) {
          acc = mfma32<MK>(acc, &ah, &bl);
          acc = mfma32<MK>(acc, &al, &bh);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          ssd = fmaf(a[e], a[e], ssd);
          if (t0 == 0) ssq = fmaf(b[e], b[e], ssq);
        }
      }
      // doc row l32's scale (or -inf for an invalid row) to the accumulator
      // layout: element i of lane l is row 8 (i / 4) + 4 h + i % 4
      {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ssd), __float_as_uint(ssd), false, false);
        const float ss = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        const float sc = norm_d ? inv_norm(ss) : 1.f;
        if (h == 0) s_sc[wl][l32] = rv ? sc : NEG_INF;
      }
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const f32x4 sc4 = *(const f32x4*)&s_sc[wl][8 * jj + 4 * h];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float sc = sc4[t];
          const float v = sc == NEG_INF ? NEG_INF : acc[4 * jj + t] * sc;
          // NaN propagates into m (the row then scores 0); the winner
          // index moves only on a strictly larger value
          if (arow && v > m) mi = (int)(t0 + 8 * jj + 4 * h + t);
          m = max_nan(m, v);
        }
      }
    }
    // column l32: max over both halves' rows, query scale, validity, sum
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    float mm = max_nan(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    if (arow) {
      // winner over lanes l, l^32: larger value, equal values the lower row;
      // -1 where the max is not finite (the row contributes 0)
      const auto si = __builtin_amdgcn_permlane32_swap((uint32_t)mi, (uint32_t)mi, false, false);
      const float v0 = __uint_as_float(sw[0]), v1 = __uint_as_float(sw[1]);
      const int i0 = (int)si[0], i1 = (int)si[1];
      const bool take1 = v1 > v0 || (v1 == v0 && (unsigned)i1 < (unsigned)i0);
      if (h == 0 && qt < lq && qt < p.amax_ld) arow[qt] = __builtin_isfinite(mm) ? (take1 ? i1 : i0) : -1;
    }
    if (norm_q) {
      const auto sq = __builtin_amdgcn_permlane32_swap(__float_as_uint(ssq), __float_as_uint(ssq), false, false);
      mm *= inv_norm(__uint_as_float(sq[0]) + __uint_as_float(sq[1]));
    }
    float v = (h == 0 && qv && __builtin_isfinite(mm)) ? mm : 0.f;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o);
    total += v;
  }
  if (lane == 0) {
    if (p.pair_q) p.out[w * p.osq] = total * p.out_scale;
    else p.out[q * p.osq + jl * p.osd] = total * p.out_scale;
  }
}

int launch_maxsim_wide(int dtype, const Params& p, hipStream_t s) {
  const int64_t waves = p.pair_q ? p.nunits : p.q.n * p.ndocs_pg;
  const int64_t nb = (waves + 3) / 4;
  if (nb > 0x7fffffffLL) return LIK_ERR_UNSUPPORTED;
  if (dtype == LIK_BF16)
    launch_kernel(maxsim_wide_kernel<EK_BF16>, dim3((unsigned)nb), dim3(256), 0, s, p);
  else if (dtype == LIK_F16)
    launch_kernel(maxsim_wide_kernel<EK_F16>, dim3((unsigned)nb), dim3(256), 0, s, p);
  else if (dtype == LIK_F32)
    launch_kernel(maxsim_wide_kernel<EK_F32>, dim3((unsigned)nb), dim3(256), 0, s, p);
  else
    return LIK_ERR_UNSUPPORTED;
  return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
}

}  // namespace lik
