// MaxSim backward for gfx950: gradients of the scores with respect to the
// (unnormalised) query and document token embeddings, from the argmax the
// training forward saved.
//
// score[i,j] = sum_s qm[i,s] * <Qh[i,s], Dh[j, a(i,j,s)]>, a = argmax (or -1:
// no valid doc token, the row contributes 0), Xh = X / max(||X||, 1e-12) when
// normalising, else X. With G = dL/dscore:
//   dL/dQh[i,s] = qm[i,s] * sum_j G[i,j] * Dh[j, a(i,j,s)]
//   dL/dDh[j,t] = sum_{i,s : a(i,j,s) = t} qm[i,s] * G[i,j] * Qh[i,s]
// and through the normalisation dL/dX = (dL/dXh - <dL/dXh, Xh> Xh) / max(||X||, 1e-12).
// This is the math of the reference's backward (backward/unified.py:27-88,
// autograd.py:183-229); the kernels are our own:
//
// * grad_q_kernel: one wavefront per query token (i, s); lanes own d/64
//   embedding dims. The argmax and G entries of 64 docs are loaded at once
//   (one per lane) and walked in doc order, so the sum order is fixed. With
//   few query tokens (small Nq) the docs are split into fixed chunks, one
//   wavefront per (chunk, token), and grad_q_finish_kernel adds the chunks'
//   partial rows in chunk order: still a fixed order.
// * grad_d_kernel: one wavefront per (doc j, block of RB doc tokens) with an
//   LDS accumulator of RB rows. It scans the (i, s) pairs in order, 64 query
//   tokens per ballot; each pair whose winner falls in the block adds its
//   scaled query row to that accumulator row. No atomics: every lane updates
//   only its own dims, in scan order, so grad_D is bitwise deterministic.
//   Packed docs (cu_seqlens): a block is RB consecutive packed rows and may
//   span several docs; it scans each of them in doc order.
//   Two layouts take other grad_D kernels with the same sums (same order):
//   the KD layout and cross products with <= 64 (query, token) pairs
//   (grad_d_kd_kernel: a doc's winners come from <= 64 pairs, so one
//   workgroup per doc) and cross products with >= 8192
//   (query, token) pairs (grad_d_sorted_kernel over the winner entries
//   radix-sorted by doc row).
// Packed queries: the wave of (i, s) exits when s is past query i's length;
// rows are addressed through cu_q (reference varlen.py:143-263).
// Pair lists (reference score_pairs.py:344-420): the score units are pairs p =
// (pair_q[p], pair_d[p]) instead of the (i, j) grid. The host builds, with a
// stable radix sort, each query's and each doc's pair list in increasing p;
// grad_q walks query i's list, grad_d doc j's list, so the order is fixed.
// Both apply the normalisation Jacobian to the finished row in registers.
#include "lik_common.h"

#include <hipcub/hipcub.hpp>

namespace lik {

template <int EK>
__device__ __forceinline__ float load_elem(const char* row, int e) {
  if constexpr (EK == EK_BF16) return __uint_as_float((uint32_t)(*(const uint16_t*)(row + 2 * e)) << 16);
  else if constexpr (EK == EK_F16) return f16_to_f32(*(const uint16_t*)(row + 2 * e));
  else return *(const float*)(row + 4 * e);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

template <int EK>
constexpr int sizeof_ek() { return EK == EK_F32 ? 4 : 2; }

struct BwdParams {
  const float* grad;  // [Nq, ld_g]
  int64_t ld_g;
  const char* q;      // Q rows: q + i*q_sn + s*q_sl, or q + (q_cu[i] + s)*q_sl when packed (bytes)
  int64_t q_sn, q_sl;
  const int32_t* q_cu;
  const char* d;      // D rows: d + j*d_sn + t*d_sl, or d + (d_cu[j] + t)*d_sl when packed (bytes)
  int64_t d_sn, d_sl;
  const int32_t* d_cu;
  const int32_t* amax;  // [Nq * ndoc_pg, Lq]
  const int8_t* qmask;  // [Nq, Lq] keep flags, or null
  int64_t qm_sn, qm_sl;
  const float* qinv;  // [Nq * Lq] inverse norms (normalise), else null
  const float* dinv;  // [Nd * Ld]
  char* gq;           // [Nq, Lq, dim] (packed: [rows, dim]) in the input dtype
  char* gd;           // [Nd, Ld, dim] (packed: [rows, dim]) in the input dtype
  int64_t nq, lq, nd, ld;  // lq / ld: padded lengths, or the longest sequence when packed
  int64_t ndoc_pg;    // docs per query: Nd (cross product) or K (KD layout)
  // pair lists (null outside pair mode): grad / argmax rows are indexed by pair
  const int32_t* pair_q;
  const int32_t* pair_d;
  const int32_t* q_ptr;   // [nq + 1] offsets into q_list
  const int32_t* q_list;  // pairs grouped by query, increasing within a query
  const int32_t* d_ptr;   // [nd + 1]
  const int32_t* d_list;
  int kd;
  int dim;
  // grad_q split over docs (dense layouts only): split c of a query token
  // walks units [c * qchunk, (c + 1) * qchunk) and leaves its fp32 partial
  // row in gq_part[c][token][64 * DPL]; grad_q_finish_kernel adds the splits
  // in order. qsplit == 1: one wavefront walks all units and stores grad_q.
  float* gq_part;
  int64_t qchunk;
  int qsplit;
  // cross-product grad_D from winner entries sorted by doc row (null: the
  // row-block kernel): entries row_vals[row_ptr[r] .. row_ptr[r + 1]) of row r
  const int32_t* row_ptr;
  const int32_t* row_vals;
};

// inv[r] = 1 / max(||row r||, 1e-12) for rows r = i*L + t of a [n, L, dim]
// tensor: LPR lanes per row, each summing 16-byte chunks, then an xor-shuffle
// reduction over the row's lanes (coalesced: a row is read as contiguous chunks).
template <int EK, int LPR>
__global__ void __launch_bounds__(256) row_invnorm_kernel(const char* x, int64_t sn, int64_t sl, int64_t n,
                                                          int64_t L, int dim, float* inv) {
  constexpr int EPC = EK == EK_F32 ? 4 : 8;  // elements per 16-byte chunk
  const int64_t r = ((int64_t)blockIdx.x * 256 + threadIdx.x) / LPR;
  const int c0 = threadIdx.x % LPR;
  const bool ok = r < n * L;
  float ss = 0.f;
  if (ok) {
    const char* row = x + (r / L) * sn + (r % L) * sl;
    for (int c = c0; c * EPC < dim; c += LPR) {
      const u32x4 v = *(const u32x4*)(row + (int64_t)c * 16);
      ss += chunk_sumsq<EK>(v);
    }
  }
#pragma unroll
  for (int o = 1; o < LPR; o <<= 1) ss += __shfl_xor(ss, o);
  if (ok && c0 == 0) inv[r] = inv_norm(ss);
}

// The same inverse norms for the winning doc rows only (sparse winners, as in
// the KD layout, where most doc rows win no max): entry w of the argmax array
// [Nq * docs, Lq] names row a of doc j; the rows no entry names are never read
// by the gradient kernels. Same lanes, chunk order and reduction as
// row_invnorm_kernel, so the same values; a row named twice is written twice
// with the same value.
template <int EK, int LPR>
__global__ void __launch_bounds__(256) winner_invnorm_kernel(const char* x, int64_t sn, int64_t sl, int64_t L,
                                                             const int32_t* amax, int64_t nw, int64_t lq,
                                                             int64_t ndoc_pg, int kd, int dim, float* inv) {
  constexpr int EPC = EK == EK_F32 ? 4 : 8;
  const int64_t w = ((int64_t)blockIdx.x * 256 + threadIdx.x) / LPR;
  const int c0 = threadIdx.x % LPR;
  int a = -1;
  int64_t j = 0;
  if (w < nw) {
    a = amax[w];
    const int64_t unit = w / lq;  // i * ndoc_pg + jl
    const int64_t i = unit / ndoc_pg, jl = unit - i * ndoc_pg;
    j = kd ? i * ndoc_pg + jl : jl;
  }
  const bool ok = a >= 0 && a < L;
  float ss = 0.f;
  if (ok) {
    const char* row = x + j * sn + (int64_t)a * sl;
    for (int c = c0; c * EPC < dim; c += LPR) {
      const u32x4 v = *(const u32x4*)(row + (int64_t)c * 16);
      ss += chunk_sumsq<EK>(v);
    }
  }
#pragma unroll
  for (int o = 1; o < LPR; o <<= 1) ss += __shfl_xor(ss, o);
  if (ok && c0 == 0) inv[j * L + a] = inv_norm(ss);
}

// Store a gradient value in the input dtype.
template <int EK>
__device__ __forceinline__ void store_elem(char* row, int e, float v) {
  if constexpr (EK == EK_BF16) *(uint16_t*)(row + 2 * e) = (uint16_t)f32_to_bf16_bits(v);
  else if constexpr (EK == EK_F16) *(uint16_t*)(row + 2 * e) = (uint16_t)f32_to_f16_bits(v);
  else *(float*)(row + 4 * e) = v;
}

// x[k] = row[e0 + k], k < DPL: the DPL elements of one lane loaded at once
// (rows start on 16-byte boundaries and e0 = lane * DPL, so the load is
// aligned to its size), elements at or past dim read as 0.
template <int EK, int DPL>
__device__ __forceinline__ void load_lane(float* x, const char* row, int e0, int dim) {
  constexpr int EB = sizeof_ek<EK>();
  if (e0 + DPL <= dim) {
    const char* p = row + (int64_t)e0 * EB;
    if constexpr (DPL * EB == 2) {
      x[0] = load_elem<EK>(row, e0);
    } else if constexpr (DPL * EB == 4) {
      const uint32_t w = *(const uint32_t*)p;
      if constexpr (EK == EK_F32) x[0] = __uint_as_float(w);
      else if constexpr (EK == EK_BF16) { x[0] = bf16lo_to_f32(w); x[1] = bf16hi_to_f32(w); }
      else { x[0] = f16_to_f32((uint16_t)(w & 0xffffu)); x[1] = f16_to_f32((uint16_t)(w >> 16)); }
    } else {
      constexpr int NW = DPL * EB / 4;  // 32-bit words, loaded 8 / 16 bytes at a time
      uint32_t w[NW];
#pragma unroll
      for (int v = 0; v < NW; v += (NW >= 4 ? 4 : 2)) {
        if constexpr (NW >= 4) {
          const u32x4 t = *(const u32x4*)(p + 4 * v);
          w[v] = t[0]; w[v + 1] = t[1]; w[v + 2] = t[2]; w[v + 3] = t[3];
        } else {
          const u32x2 t = *(const u32x2*)(p + 4 * v);
          w[v] = t[0]; w[v + 1] = t[1];
        }
      }
#pragma unroll
      for (int k = 0; k < DPL; ++k) {
        if constexpr (EK == EK_F32) x[k] = __uint_as_float(w[k]);
        else if constexpr (EK == EK_BF16) x[k] = (k & 1) ? bf16hi_to_f32(w[k >> 1]) : bf16lo_to_f32(w[k >> 1]);
        else x[k] = f16_to_f32((uint16_t)((k & 1) ? (w[k >> 1] >> 16) : (w[k >> 1] & 0xffffu)));
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < DPL; ++k) x[k] = e0 + k < dim ? load_elem<EK>(row, e0 + k) : 0.f;
  }
}

// acc[k] += c * row[e0 + k], k < DPL
template <int EK, int DPL>
__device__ __forceinline__ void axpy_lane(float* acc, const char* row, int e0, int dim, float c) {
  float x[DPL];
  load_lane<EK, DPL>(x, row, e0, dim);
#pragma unroll
  for (int k = 0; k < DPL; ++k) acc[k] = fmaf(c, x[k], acc[k]);
}

// Query token w = i * lq + s: its storage row (packed queries: through cu_q),
// or -1 when s is past query i's length.
__device__ __forceinline__ int64_t grad_q_row(const BwdParams& bp, int64_t i, int64_t s, int64_t w) {
  if (!bp.q_cu) return w;
  const int64_t q0 = bp.q_cu[i];
  return s < (int64_t)bp.q_cu[i + 1] - q0 ? q0 + s : -1;
}

// Query mask, the normalisation Jacobian on the finished row, store.
template <int EK, int DPL>
__device__ __forceinline__ void grad_q_store(const BwdParams& bp, int64_t i, int64_t s, int64_t qr, float* acc,
                                             int lane) {
  const bool keep = !bp.qmask || bp.qmask[i * bp.qm_sn + s * bp.qm_sl] != 0;
  if (bp.qinv) {
    const float qi = bp.qinv[qr];
    const char* qrow = bp.q_cu ? bp.q + qr * bp.q_sl : bp.q + i * bp.q_sn + s * bp.q_sl;
    float xh[DPL], dot = 0.f;
#pragma unroll
    for (int k = 0; k < DPL; ++k) {
      const int e = lane * DPL + k;
      xh[k] = e < bp.dim ? load_elem<EK>(qrow, e) * qi : 0.f;
      dot = fmaf(acc[k], xh[k], dot);
    }
    dot = wave_sum(dot);
#pragma unroll
    for (int k = 0; k < DPL; ++k) acc[k] = (acc[k] - dot * xh[k]) * qi;
  }
  char* out = bp.gq + qr * bp.dim * (int64_t)sizeof_ek<EK>();
#pragma unroll
  for (int k = 0; k < DPL; ++k) {
    const int e = lane * DPL + k;
    if (e < bp.dim) store_elem<EK>(out, e, keep ? acc[k] : 0.f);
  }
}

template <int EK, int DPL>
__global__ void __launch_bounds__(256) grad_q_kernel(const BwdParams bp) {
  const int lane = threadIdx.x & 63;
  const int64_t nwt = bp.nq * bp.lq;
  int64_t w = __builtin_amdgcn_readfirstlane((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6));
  if (w >= nwt * bp.qsplit) return;
  const int64_t c = w / nwt;  // doc split
  w -= c * nwt;
  const int64_t i = w / bp.lq, s = w % bp.lq;
  const int64_t qr = grad_q_row(bp, i, s, w);  // storage row of token (i, s)
  if (qr < 0) return;
  const int64_t j0 = bp.kd ? i * bp.ndoc_pg : 0;
  // units of query i: docs jl < ndoc_pg, or its pairs q_list[u0 .. u0 + nu)
  int64_t nu = bp.ndoc_pg, u0 = 0;
  if (bp.q_ptr) {
    u0 = bp.q_ptr[i];
    nu = (int64_t)bp.q_ptr[i + 1] - u0;
  }
  int64_t ub = 0, ue = nu;
  if (bp.qsplit > 1) {
    ub = c * bp.qchunk;
    ue = ub + bp.qchunk < nu ? ub + bp.qchunk : nu;
  }
  float acc[DPL];
#pragma unroll
  for (int k = 0; k < DPL; ++k) acc[k] = 0.f;
  for (int64_t c0 = ub; c0 < ue; c0 += 64) {
    const int64_t jl = c0 + lane;
    int av = -1, jd = 0;
    float gv = 0.f;
    if (jl < ue) {
      if (bp.q_ptr) {
        const int64_t pr = bp.q_list[u0 + jl];
        av = bp.amax[pr * bp.lq + s];
        gv = bp.grad[pr];
        jd = bp.pair_d[pr];
      } else {
        av = bp.amax[(i * bp.ndoc_pg + jl) * bp.lq + s];
        gv = bp.grad[i * bp.ld_g + jl];
        jd = (int)(j0 + jl);
      }
    }
    float sv = gv;
    if (bp.dinv && av >= 0) sv *= bp.dinv[(int64_t)jd * bp.ld + av];  // dinv only for padded docs
    uint64_t bal = __ballot(av >= 0 && gv != 0.f);
    // up to HB winning rows loaded before any is added (one memory latency
    // per batch instead of one per doc), added in doc order
    constexpr int HB = DPL <= 2 ? 8 : (DPL == 4 ? 4 : (DPL == 8 ? 2 : 1));
    while (bal) {
      float xs[HB][DPL], scs[HB];
      int nb = 0;
#pragma unroll
      for (int b = 0; b < HB; ++b) {
        if (bal) {
          const int l = __builtin_ctzll(bal);
          bal &= bal - 1;
          const int a = __builtin_amdgcn_readlane(av, l);
          scs[b] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sv), l));
          const int64_t jg = __builtin_amdgcn_readlane(jd, l);
          const char* row = bp.d_cu ? bp.d + ((int64_t)bp.d_cu[jg] + a) * bp.d_sl
                                    : bp.d + jg * bp.d_sn + (int64_t)a * bp.d_sl;
          load_lane<EK, DPL>(xs[b], row, lane * DPL, bp.dim);
          nb = b + 1;
        }
      }
#pragma unroll
      for (int b = 0; b < HB; ++b) {
        if (b >= nb) break;
#pragma unroll
        for (int k = 0; k < DPL; ++k) acc[k] = fmaf(scs[b], xs[b][k], acc[k]);
      }
    }
  }
  if (bp.qsplit > 1) {
    float* part = bp.gq_part + ((c * nwt + w) * 64 + lane) * DPL;
#pragma unroll
    for (int k = 0; k < DPL; ++k) part[k] = acc[k];
    return;
  }
  grad_q_store<EK, DPL>(bp, i, s, qr, acc, lane);
}

// Sum of the doc splits' partial rows, in split order, then the store.
template <int EK, int DPL>
__global__ void __launch_bounds__(256) grad_q_finish_kernel(const BwdParams bp) {
  const int lane = threadIdx.x & 63;
  const int64_t nwt = bp.nq * bp.lq;
  const int64_t w = __builtin_amdgcn_readfirstlane((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6));
  if (w >= nwt) return;
  const int64_t i = w / bp.lq, s = w % bp.lq;
  const int64_t qr = grad_q_row(bp, i, s, w);
  if (qr < 0) return;
  float acc[DPL];
#pragma unroll
  for (int k = 0; k < DPL; ++k) acc[k] = 0.f;
  for (int c = 0; c < bp.qsplit; ++c) {
    const float* part = bp.gq_part + ((c * nwt + w) * 64 + lane) * DPL;
#pragma unroll
    for (int k = 0; k < DPL; ++k) acc[k] += part[k];
  }
  grad_q_store<EK, DPL>(bp, i, s, qr, acc, lane);
}

// Doc rows per grad_d block: every block rescans all the (i, s) pairs of its
// doc, but the scan is latency-bound, so more, shorter blocks (more waves per
// CU) win: 16 rows measured best for up to 2 dims per lane (8 KB of
// accumulator; 8 and 32 rows slower, 64 much slower), 64 / DPL rows beyond.
template <int DPL>
constexpr int grad_d_rows() { return DPL <= 2 ? 16 : (64 / DPL < 32 ? 64 / DPL : 32); }

// RB doc rows per wavefront, RB * 64 * DPL floats of LDS accumulator.
// Padded docs: block b is rows [t0, t0 + RB) of doc b / nrb. Packed docs: block
// b is storage rows [cu[0] + b*RB, +RB), each doc overlapping it scanned in turn.
template <int EK, int DPL>
__global__ void __launch_bounds__(64) grad_d_kernel(const BwdParams bp) {
  constexpr int RB = grad_d_rows<DPL>();
  __shared__ __attribute__((aligned(16))) float s_acc[RB][64 * DPL];
  const int lane = threadIdx.x;
#pragma unroll
  for (int r = 0; r < RB; ++r)
#pragma unroll
    for (int k = 0; k < DPL; ++k) s_acc[r][lane * DPL + k] = 0.f;
  uint64_t touched = 0;  // rows of the block that received a contribution (wave-uniform)

  // Add the contributions of doc j whose winner a lies in [wlo, wlo + n) to
  // accumulator rows off + (a - wlo).
  auto scan_doc = [&](int64_t j, int64_t wlo, int n, int off) {
    // units of doc j: queries i (grid / KD), or its pairs d_list[u_begin .. u_end)
    const int64_t jl = bp.kd ? j % bp.ndoc_pg : j;
    int64_t u_begin = bp.kd ? j / bp.ndoc_pg : 0;
    int64_t u_end = bp.kd ? u_begin + 1 : bp.nq;
    if (bp.d_ptr) {
      u_begin = bp.d_ptr[j];
      u_end = bp.d_ptr[j + 1];
    }
    if (!bp.d_ptr && !bp.q_cu && bp.lq < 64) {
      // Short padded queries on the (i, j) grid: the (i, s) pairs of units
      // [u_begin, u_end) flattened, 64 per pass (one query per pass would
      // leave lanes idle), the next pass's argmax / G / scale loads issued
      // before this pass's hits are added. Same pair order as the per-query
      // loop below, so the same sums. Lane (i, s) advances by 64 per pass.
      const int64_t f0 = u_begin * bp.lq, f1 = u_end * bp.lq;
      int64_t li = u_begin + lane / bp.lq, ls = lane % bp.lq;  // pair f0 + lane
      auto load_pass = [&](int64_t fb, int& a, float& sc, int64_t& qoff) {
        const int64_t f = fb + lane;
        const int64_t i = li, s = ls;
        ls += 64;
        while (ls >= bp.lq) {
          ls -= bp.lq;
          ++li;
        }
        a = -1;
        sc = 0.f;
        qoff = 0;
        if (f < f1) {
          // independent loads (no load waits on another), so a pass costs one
          // memory latency; a zero G or a masked query token drops the pair
          const float gij = bp.grad[i * bp.ld_g + jl];
          int av = bp.amax[(i * bp.ndoc_pg + jl) * bp.lq + s];
          const bool keep = !bp.qmask || bp.qmask[i * bp.qm_sn + s * bp.qm_sl] != 0;
          const float qi = bp.qinv ? bp.qinv[i * bp.lq + s] : 1.f;
          if (gij == 0.f || !keep) av = -1;
          a = av;
          sc = bp.qinv ? gij * qi : gij;
          qoff = i * bp.q_sn + s * bp.q_sl;
        }
      };
      int a_c, a_n;
      float sc_c, sc_n;
      int64_t qo_c, qo_n;
      load_pass(f0, a_c, sc_c, qo_c);
      for (int64_t fb = f0; fb < f1; fb += 64) {
        load_pass(fb + 64, a_n, sc_n, qo_n);
        uint64_t bal = __ballot(a_c >= wlo && a_c < wlo + n);
        while (bal) {
          const int l = __builtin_ctzll(bal);
          bal &= bal - 1;
          const int r = off + __builtin_amdgcn_readlane(a_c, l) - (int)wlo;
          touched |= 1ull << r;
          const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc_c), l));
          const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)qo_c, l);
          const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)qo_c >> 32), l);
          const char* qrow = bp.q + (int64_t)(((uint64_t)hi << 32) | lo);
          // this lane's DPL dims of row r: one LDS read, one write (the
          // elements past dim accumulate zeros and are never stored)
          float* ar = &s_acc[r][lane * DPL];
          float av[DPL];
#pragma unroll
          for (int k = 0; k < DPL; ++k) av[k] = ar[k];
          axpy_lane<EK, DPL>(av, qrow, lane * DPL, bp.dim, c);
#pragma unroll
          for (int k = 0; k < DPL; ++k) ar[k] = av[k];
        }
        a_c = a_n;
        sc_c = sc_n;
        qo_c = qo_n;
      }
      return;
    }
    for (int64_t u = u_begin; u < u_end; ++u) {
      int64_t i, arow;
      float gij;
      if (bp.d_ptr) {
        arow = bp.d_list[u];
        i = bp.pair_q[arow];
        gij = bp.grad[arow];
      } else {
        i = u;
        arow = i * bp.ndoc_pg + jl;
        gij = bp.grad[i * bp.ld_g + jl];
      }
      if (gij == 0.f) continue;
      const int32_t* am = bp.amax + arow * bp.lq;
      int64_t qlen = bp.lq, qbase = 0;
      if (bp.q_cu) {
        qbase = bp.q_cu[i];
        qlen = (int64_t)bp.q_cu[i + 1] - qbase;
      }
      for (int64_t s0 = 0; s0 < qlen; s0 += 64) {
        const int64_t s = s0 + lane;
        int a = s < qlen ? am[s] : -1;
        if (a >= 0 && bp.qmask && bp.qmask[i * bp.qm_sn + s * bp.qm_sl] == 0) a = -1;
        float sc = gij;
        if (bp.qinv && a >= 0) sc *= bp.qinv[bp.q_cu ? qbase + s : i * bp.lq + s];
        uint64_t bal = __ballot(a >= wlo && a < wlo + n);
        while (bal) {
          const int l = __builtin_ctzll(bal);
          bal &= bal - 1;
          const int r = off + __builtin_amdgcn_readlane(a, l) - (int)wlo;
          touched |= 1ull << r;
          const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc), l));
          const char* qrow = bp.q_cu ? bp.q + (qbase + s0 + l) * bp.q_sl : bp.q + i * bp.q_sn + (s0 + l) * bp.q_sl;
          // this lane's DPL dims of row r: one LDS read, one write (the
          // elements past dim accumulate zeros and are never stored)
          float* ar = &s_acc[r][lane * DPL];
          float av[DPL];
#pragma unroll
          for (int k = 0; k < DPL; ++k) av[k] = ar[k];
          axpy_lane<EK, DPL>(av, qrow, lane * DPL, bp.dim, c);
#pragma unroll
          for (int k = 0; k < DPL; ++k) ar[k] = av[k];
        }
      }
    }
  };

  int nrows;         // rows of this block
  int64_t out_row0;  // storage row of accumulator row 0
  int64_t j_pad = 0, t0 = 0;
  if (bp.d_cu) {
    const int64_t base = bp.d_cu[0], endr = bp.d_cu[bp.nd];
    const int64_t r0 = base + (int64_t)blockIdx.x * RB;
    if (r0 >= endr) return;
    nrows = (int)(endr - r0 < RB ? endr - r0 : RB);
    out_row0 = r0;
    // first doc whose rows reach past r0: largest j with cu[j] <= r0 (binary search)
    int64_t lo = 0, hi = bp.nd;  // invariant: cu[lo] <= r0 < cu[hi]
    while (hi - lo > 1) {
      const int64_t mid = (lo + hi) >> 1;
      if (bp.d_cu[mid] <= r0) lo = mid;
      else hi = mid;
    }
    for (int64_t j = lo; j < bp.nd; ++j) {
      const int64_t c0 = bp.d_cu[j], c1 = bp.d_cu[j + 1];
      if (c0 >= r0 + nrows) break;
      const int64_t a0 = r0 > c0 ? r0 : c0;  // overlap [a0, a1) in storage rows
      const int64_t a1 = c1 < r0 + nrows ? c1 : r0 + nrows;
      if (a1 > a0) scan_doc(j, a0 - c0, (int)(a1 - a0), (int)(a0 - r0));
    }
  } else {
    const int64_t nrb = (bp.ld + RB - 1) / RB;
    j_pad = blockIdx.x / nrb;
    t0 = (blockIdx.x % nrb) * RB;
    nrows = (int)(bp.ld - t0 < RB ? bp.ld - t0 : RB);
    out_row0 = j_pad * bp.ld + t0;
    scan_doc(j_pad, t0, nrows, 0);
  }

  // finished rows: normalisation Jacobian (padded docs only), then store
  for (int r = 0; r < nrows; ++r) {
    char* out = bp.gd + (out_row0 + r) * bp.dim * (int64_t)sizeof_ek<EK>();
    if (!((touched >> r) & 1ull)) {  // no winner in this row: zero gradient, no D read
#pragma unroll
      for (int k = 0; k < DPL; ++k) {
        const int e = lane * DPL + k;
        if (e < bp.dim) store_elem<EK>(out, e, 0.f);
      }
      continue;
    }
    float gh[DPL];
#pragma unroll
    for (int k = 0; k < DPL; ++k) gh[k] = s_acc[r][lane * DPL + k];
    if (bp.dinv) {
      const int64_t t = t0 + r;
      const float di = bp.dinv[j_pad * bp.ld + t];
      const char* drow = bp.d + j_pad * bp.d_sn + t * bp.d_sl;
      float xh[DPL], dot = 0.f;
#pragma unroll
      for (int k = 0; k < DPL; ++k) {
        const int e = lane * DPL + k;
        xh[k] = e < bp.dim ? load_elem<EK>(drow, e) * di : 0.f;
        dot = fmaf(gh[k], xh[k], dot);
      }
      dot = wave_sum(dot);
#pragma unroll
      for (int k = 0; k < DPL; ++k) gh[k] = (gh[k] - dot * xh[k]) * di;
    }
#pragma unroll
    for (int k = 0; k < DPL; ++k) {
      const int e = lane * DPL + k;
      if (e < bp.dim) store_elem<EK>(out, e, gh[k]);
    }
  }
}

// KD layout (padded docs and queries, Lq <= 64): doc j belongs to query
// i = j / K alone, so its gradient rows are the (at most Lq) rows that won one
// of query i's tokens; likewise a cross product with Nq * Lq <= 64 (a doc's
// winners come from those <= 64 pairs). One workgroup of 4 wavefronts per
// doc: in each, lane s holds pair s's winner; distinct winning row number k (in order of first
// token) is summed by wavefront k % 4, adding its tokens' scaled query rows in
// increasing s (the order of grad_d_kernel's scan, so the same sums), then
// takes the normalise Jacobian and is stored. The doc's other rows are
// written as zeros by the whole workgroup (each wavefront builds the bitmap of
// winning rows in its own LDS words). No per-block rescans of the pairs, one
// streaming pass of stores over the doc.
constexpr int KD_GD_MAXLD = 8192;
template <int EK, int DPL>
__global__ void __launch_bounds__(256) grad_d_kd_kernel(const BwdParams bp) {
  __shared__ uint32_t s_hit[4][KD_GD_MAXLD / 32];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t j = blockIdx.x;
  const int nwords = (int)((bp.ld + 31) / 32);
  for (int w = lane; w < nwords; w += 64) s_hit[wv][w] = 0u;
  // lane f: KD, token f of doc j's query; cross product (Nq * Lq <= 64), the
  // pair (i, s) = (f / Lq, f % Lq) (the row-block kernel's scan order)
  const int64_t i = bp.kd ? j / bp.ndoc_pg : lane / bp.lq;
  const int64_t jl = bp.kd ? j - i * bp.ndoc_pg : j;
  const int64_t sl = bp.kd ? lane : lane - i * bp.lq;
  const int64_t npair = bp.kd ? bp.lq : bp.nq * bp.lq;
  int a = -1;
  float sc = 0.f;
  int64_t qoff = 0;
  if (lane < npair) {
    const float gij = bp.grad[i * bp.ld_g + jl];
    if (gij != 0.f) {
      a = bp.amax[(i * bp.ndoc_pg + jl) * bp.lq + sl];
      if (bp.qmask && bp.qmask[i * bp.qm_sn + sl * bp.qm_sl] == 0) a = -1;
      sc = bp.qinv ? gij * bp.qinv[i * bp.lq + sl] : gij;
      qoff = i * bp.q_sn + sl * bp.q_sl;
    }
  }
  const int64_t esz = sizeof_ek<EK>();
  const int64_t rowb = (int64_t)bp.dim * esz;
  char* gdoc = bp.gd + j * bp.ld * rowb;
  uint64_t todo = __ballot(a >= 0);
  for (int k = 0; todo; ++k) {
    const int t = __builtin_amdgcn_readlane(a, __builtin_ctzll(todo));
    uint64_t same = __ballot(a == t);
    todo &= ~same;
    if (lane == 0) s_hit[wv][t >> 5] |= 1u << (t & 31);
    if ((k & 3) != wv) continue;
    float gh[DPL];
#pragma unroll
    for (int e = 0; e < DPL; ++e) gh[e] = 0.f;
    while (same) {
      const int l = __builtin_ctzll(same);
      same &= same - 1;
      const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc), l));
      const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)qoff, l);
      const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)qoff >> 32), l);
      axpy_lane<EK, DPL>(gh, bp.q + (int64_t)(((uint64_t)hi << 32) | lo), lane * DPL, bp.dim, c);
    }
    if (bp.dinv) {
      const float di = bp.dinv[j * bp.ld + t];
      const char* drow = bp.d + j * bp.d_sn + (int64_t)t * bp.d_sl;
      float xh[DPL], dot = 0.f;
#pragma unroll
      for (int e = 0; e < DPL; ++e) {
        const int el = lane * DPL + e;
        xh[e] = el < bp.dim ? load_elem<EK>(drow, el) * di : 0.f;
        dot = fmaf(gh[e], xh[e], dot);
      }
      dot = wave_sum(dot);
#pragma unroll
      for (int e = 0; e < DPL; ++e) gh[e] = (gh[e] - dot * xh[e]) * di;
    }
    char* out = gdoc + (int64_t)t * rowb;
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      const int el = lane * DPL + e;
      if (el < bp.dim) store_elem<EK>(out, el, gh[e]);
    }
  }
  // the rows no token won: zeros, 16 bytes per thread per store (LDS
  // operations of one wavefront complete in order: its bitmap is final)
  const int64_t nchunk = bp.ld * rowb / 16;
  const int64_t cpr = rowb / 16;
  for (int64_t c = threadIdx.x; c < nchunk; c += 256) {
    const int64_t t = c / cpr;
    if (!((s_hit[wv][t >> 5] >> (t & 31)) & 1u)) *(u32x4*)(gdoc + c * 16) = u32x4{0u, 0u, 0u, 0u};
  }
}

// Cross-product layout with many (query, token) pairs per doc: instead of
// row blocks that each rescan all Nq * Lq pairs, the winner entries
// f = (i * Nd + j) * Lq + s are sorted once by doc row j * Ld + a (a stable
// radix sort, so a row's entries stay in increasing (i, s): the row-block
// kernel's scan order, hence the same sums). Entries that add nothing (no
// winner, G = 0, a masked query token) get the key Nd * Ld and sort last.
__global__ void __launch_bounds__(256) row_keys_kernel(const BwdParams bp, int64_t n, int32_t* keys, int32_t* vals) {
  const int64_t f = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (f >= n) return;
  const int64_t s = f % bp.lq, ij = f / bp.lq;
  const int64_t j = ij % bp.nd, i = ij / bp.nd;
  const int a = bp.amax[f];
  const bool keep = a >= 0 && bp.grad[i * bp.ld_g + j] != 0.f && (!bp.qmask || bp.qmask[i * bp.qm_sn + s * bp.qm_sl] != 0);
  keys[f] = keep ? (int32_t)(j * bp.ld + a) : (int32_t)(bp.nd * bp.ld);
  vals[f] = (int32_t)f;
}

// One wavefront per doc row: its sorted entries added in order (scaled query
// rows, as grad_d_kernel adds them), the normalise Jacobian, the store; a row
// without entries is stored as zeros.
template <int EK, int DPL>
__global__ void __launch_bounds__(256) grad_d_sorted_kernel(const BwdParams bp) {
  const int lane = threadIdx.x & 63;
  const int64_t r = __builtin_amdgcn_readfirstlane((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6));
  if (r >= bp.nd * bp.ld) return;
  const int64_t j = r / bp.ld, t = r - j * bp.ld;
  const int b = bp.row_ptr[r], e = bp.row_ptr[r + 1];
  float gh[DPL];
#pragma unroll
  for (int k = 0; k < DPL; ++k) gh[k] = 0.f;
  for (int k0 = b; k0 < e; k0 += 64) {
    float sc = 0.f;
    int64_t qoff = 0;
    if (k0 + lane < e) {
      const int64_t f = bp.row_vals[k0 + lane];
      const int64_t s = f % bp.lq, i = f / bp.lq / bp.nd;
      const float gij = bp.grad[i * bp.ld_g + j];
      sc = bp.qinv ? gij * bp.qinv[i * bp.lq + s] : gij;
      qoff = i * bp.q_sn + s * bp.q_sl;
    }
    const int m = e - k0 < 64 ? e - k0 : 64;
    for (int l = 0; l < m; ++l) {
      const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc), l));
      const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)qoff, l);
      const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)qoff >> 32), l);
      axpy_lane<EK, DPL>(gh, bp.q + (int64_t)(((uint64_t)hi << 32) | lo), lane * DPL, bp.dim, c);
    }
  }
  if (bp.dinv && e > b) {
    const float di = bp.dinv[r];
    const char* drow = bp.d + j * bp.d_sn + t * bp.d_sl;
    float xh[DPL], dot = 0.f;
#pragma unroll
    for (int k = 0; k < DPL; ++k) {
      const int el = lane * DPL + k;
      xh[k] = el < bp.dim ? load_elem<EK>(drow, el) * di : 0.f;
      dot = fmaf(gh[k], xh[k], dot);
    }
    dot = wave_sum(dot);
#pragma unroll
    for (int k = 0; k < DPL; ++k) gh[k] = (gh[k] - dot * xh[k]) * di;
  }
  char* out = bp.gd + r * bp.dim * (int64_t)sizeof_ek<EK>();
#pragma unroll
  for (int k = 0; k < DPL; ++k) {
    const int el = lane * DPL + k;
    if (el < bp.dim) store_elem<EK>(out, el, gh[k]);
  }
}

template <int EK, int DPL>
int launch_bwd(const BwdParams& bp, hipStream_t s) {
  constexpr int RB = grad_d_rows<DPL>();
  const int64_t nw = bp.nq * bp.lq;
  if (nw > 0) {
    hipLaunchKernelGGL((grad_q_kernel<EK, DPL>), dim3((unsigned)((nw * bp.qsplit + 3) / 4)), dim3(256), 0, s, bp);
    if (hipGetLastError() != hipSuccess) return LIK_ERR_LAUNCH;
    if (bp.qsplit > 1) {
      hipLaunchKernelGGL((grad_q_finish_kernel<EK, DPL>), dim3((unsigned)((nw + 3) / 4)), dim3(256), 0, s, bp);
      if (hipGetLastError() != hipSuccess) return LIK_ERR_LAUNCH;
    }
  }
  if (bp.gd && bp.row_ptr) {
    const int64_t nr = bp.nd * bp.ld;
    hipLaunchKernelGGL((grad_d_sorted_kernel<EK, DPL>), dim3((unsigned)((nr + 3) / 4)), dim3(256), 0, s, bp);
    return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
  }
  if (bp.gd && !bp.q_ptr && !bp.q_cu && !bp.d_cu && (bp.kd ? bp.lq <= 64 : bp.nq * bp.lq <= 64) &&
      bp.ld <= KD_GD_MAXLD &&
      ((int64_t)bp.dim * sizeof_ek<EK>()) % 16 == 0 && ((uintptr_t)bp.gd) % 16 == 0) {
    if (bp.nd > 0x7fffffffLL) return LIK_ERR_UNSUPPORTED;
    hipLaunchKernelGGL((grad_d_kd_kernel<EK, DPL>), dim3((unsigned)bp.nd), dim3(256), 0, s, bp);
    return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
  }
  // packed docs: sum of lengths <= nd * ld, so nd * ld / RB blocks cover them
  const int64_t nb = !bp.gd ? 0 : bp.d_cu ? (bp.nd * bp.ld + RB - 1) / RB : bp.nd * ((bp.ld + RB - 1) / RB);
  if (nb > 0x7fffffffLL) return LIK_ERR_UNSUPPORTED;
  if (nb > 0) {
    hipLaunchKernelGGL((grad_d_kernel<EK, DPL>), dim3((unsigned)nb), dim3(64), 0, s, bp);
    if (hipGetLastError() != hipSuccess) return LIK_ERR_LAUNCH;
  }
  return LIK_OK;
}

template <int EK>
int launch_bwd_dpl(const BwdParams& bp, hipStream_t s) {
  if (bp.dim <= 64) return launch_bwd<EK, 1>(bp, s);
  if (bp.dim <= 128) return launch_bwd<EK, 2>(bp, s);
  if (bp.dim <= 256) return launch_bwd<EK, 4>(bp, s);
  if (bp.dim <= 512) return launch_bwd<EK, 8>(bp, s);
  if (bp.dim <= 1024) return launch_bwd<EK, 16>(bp, s);
  if (bp.dim <= 2048) return launch_bwd<EK, 32>(bp, s);
  return LIK_ERR_UNSUPPORTED;
}

template <int EK>
int launch_invnorm(const char* x, int64_t sn, int64_t sl, int64_t n, int64_t L, int dim, float* inv, hipStream_t s) {
  constexpr int LPR = 16;  // lanes per row
  const int64_t rows = n * L;
  if (rows == 0) return LIK_OK;
  hipLaunchKernelGGL((row_invnorm_kernel<EK, LPR>), dim3((unsigned)((rows * LPR + 255) / 256)), dim3(256), 0, s, x,
                     sn, sl, n, L, dim, inv);
  return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
}

template <int EK>
int launch_winner_invnorm(const BwdParams& bp, float* inv, hipStream_t s) {
  constexpr int LPR = 16;
  const int64_t nw = bp.nq * bp.ndoc_pg * bp.lq;
  if (nw == 0) return LIK_OK;
  hipLaunchKernelGGL((winner_invnorm_kernel<EK, LPR>), dim3((unsigned)((nw * LPR + 255) / 256)), dim3(256), 0, s,
                     bp.d, bp.d_sn, bp.d_sl, bp.ld, bp.amax, nw, bp.lq, bp.ndoc_pg, bp.kd, bp.dim, inv);
  return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
}

int elem_size(int dt) { return dt == LIK_F32 ? 4 : 2; }

// Sort keys of the pair lists: key = owner (query or doc) index, or n (sorted
// last, in no list) for a pair with an out-of-range index; vals = pair index.
__global__ void __launch_bounds__(256) pair_keys_kernel(const int32_t* pair_q, const int32_t* pair_d, int64_t np,
                                                        int64_t nq, int64_t nd, int32_t* kq, int32_t* kd,
                                                        int32_t* iota) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= np) return;
  const int32_t q = pair_q[p], d = pair_d[p];
  const bool ok = q >= 0 && q < nq && d >= 0 && d < nd;
  kq[p] = ok ? q : (int32_t)nq;
  kd[p] = ok ? d : (int32_t)nd;
  iota[p] = (int32_t)p;
}

// ptr[k] = first position of key >= k in the sorted keys, k = 0 .. n.
__global__ void __launch_bounds__(256) bucket_ptr_kernel(const int32_t* sorted, int64_t np, int64_t n, int32_t* ptr) {
  const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (k > n) return;
  int64_t lo = 0, hi = np;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (sorted[mid] < k) lo = mid + 1;
    else hi = mid;
  }
  ptr[k] = (int32_t)lo;
}

struct PairWs {
  size_t kq, kd, iota, ks, qlist, dlist, qptr, dptr, temp, temp_bytes, total;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static int end_bit_for(int64_t n) {
  int b = 1;
  while (b < 31 && ((int64_t)1 << b) <= n) ++b;
  return b;
}

static PairWs pair_ws_layout(int64_t np, int64_t nq, int64_t nd) {
  PairWs w{};
  size_t o = 0;
  const size_t a = align256((size_t)np * 4);
  w.kq = o; o += a;
  w.kd = o; o += a;
  w.iota = o; o += a;
  w.ks = o; o += a;
  w.qlist = o; o += a;
  w.dlist = o; o += a;
  w.qptr = o; o += align256((size_t)(nq + 1) * 4);
  w.dptr = o; o += align256((size_t)(nd + 1) * 4);
  size_t tb = 0;
  hipcub::DeviceRadixSort::SortPairs(nullptr, tb, (const int32_t*)nullptr, (int32_t*)nullptr,
                                     (const int32_t*)nullptr, (int32_t*)nullptr, (int)np, 0,
                                     end_bit_for(nq > nd ? nq : nd));
  w.temp = o;
  w.temp_bytes = tb;
  o += align256(tb);
  w.total = o + 256;
  return w;
}

}  // namespace lik

using namespace lik;

extern "C" {

static bool bwd_norm_q(uint32_t f) { return (f & (LIK_NORMALIZE | LIK_NORMALIZE_Q)) != 0; }
static bool bwd_norm_d(uint32_t f) { return (f & (LIK_NORMALIZE | LIK_NORMALIZE_D)) != 0; }

size_t lik_maxsim_pairs_backward_workspace_size(const lik_seqs_t* Q, const lik_seqs_t* D, int64_t num_pairs) {
  if (!Q || !D || num_pairs <= 0 || Q->n < 0 || D->n < 0) return 0;
  return pair_ws_layout(num_pairs, Q->n, D->n).total;
}

// Doc splits of grad_q (dense layouts): when the query tokens alone give
// fewer than 2048 wavefronts (counting 32 tokens per query), each token's docs
// are split into chunks of >= 16 so that about 2048 wavefronts walk them. The
// split depends on Nq and the docs per query only, not on Lq, so a query
// batch padded to another length gets the same bits.
static void grad_q_split(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags, int64_t* split, int64_t* chunk) {
  *split = 1;
  *chunk = 0;
  if (Q->n <= 0 || D->n <= 0 || Q->len <= 0 || Q->dim <= 0 || Q->dim > 2048) return;
  const int64_t ndoc = (flags & LIK_KD_LAYOUT) ? D->n / Q->n : D->n;
  const int64_t want = 2048 / (32 * Q->n), most = (ndoc + 15) / 16;
  const int64_t ns = want < most ? want : most;
  if (ns <= 1) return;
  *chunk = (ndoc + ns - 1) / ns;
  *split = (ndoc + *chunk - 1) / *chunk;
}

// fp32 partial rows of the grad_q doc splits: [split][Nq * Lq][64 * DPL]
static size_t grad_q_part_bytes(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags) {
  int64_t split, chunk;
  grad_q_split(Q, D, flags, &split, &chunk);
  if (split <= 1) return 0;
  int64_t dpl = 1;
  while (dpl * 64 < Q->dim) dpl *= 2;
  return (size_t)(split * Q->n * Q->len * 64 * dpl) * sizeof(float);
}

// Sorted-entry grad_D (cross product, padded, many pairs per doc): keys and
// values in and out, the row pointers, the sort's temporary storage.
struct RowWs {
  size_t kin, vin, kout, vout, ptr, temp, temp_bytes, total;
  int64_t n, rows;
};
static RowWs row_ws_layout(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags) {
  RowWs w{};
  if ((flags & LIK_KD_LAYOUT) || Q->cu_seqlens || D->cu_seqlens || Q->n <= 0 || D->n <= 0 || Q->len <= 0 ||
      D->len <= 0)
    return w;
  const int64_t n = Q->n * D->n * Q->len, rows = D->n * D->len;
  // worth it when a row block would rescan many pairs (measured: 8192 pairs
  // per doc 0.92 -> 0.81 ms, 65,920 2.65 -> 2.21 ms, but 4096 pairs over
  // 1030-token docs 0.45 -> 0.50 ms); 32-bit entry and row ids
  if (Q->n * Q->len < 8192 || n >= ((int64_t)1 << 31) || rows >= ((int64_t)1 << 31) - 1) return w;
  size_t o = 0;
  const size_t a = align256((size_t)n * 4);
  w.kin = o; o += a;
  w.vin = o; o += a;
  w.kout = o; o += a;
  w.vout = o; o += a;
  w.ptr = o; o += align256((size_t)(rows + 1) * 4);
  size_t tb = 0;
  hipcub::DeviceRadixSort::SortPairs(nullptr, tb, (const int32_t*)nullptr, (int32_t*)nullptr,
                                     (const int32_t*)nullptr, (int32_t*)nullptr, (int)n, 0, end_bit_for(rows));
  w.temp = o;
  w.temp_bytes = tb;
  o += align256(tb);
  w.total = o;
  w.n = n;
  w.rows = rows;
  return w;
}

// float entries of the inverse-norm arrays at the start of the workspace
static size_t bwd_norm_floats(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags) {
  size_t n = 0;
  if (bwd_norm_q(flags)) n += (size_t)(Q->n * Q->len);
  if (bwd_norm_d(flags)) n += (size_t)(D->n * D->len);
  return n;
}

size_t lik_maxsim_backward_workspace_size(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags) {
  if (!Q || !D || Q->n < 0 || D->n < 0 || Q->len < 0 || D->len < 0) return 0;
  const size_t b = align256(bwd_norm_floats(Q, D, flags) * sizeof(float)) + align256(grad_q_part_bytes(Q, D, flags)) +
                   row_ws_layout(Q, D, flags).total;
  return b ? b + 256 : 0;
}

int lik_maxsim_backward(const float* grad, int64_t grad_ld, const lik_seqs_t* Q, const lik_seqs_t* D,
                        const int32_t* argmax, uint32_t flags, void* grad_q, void* grad_d, void* workspace,
                        size_t workspace_bytes, lik_stream_t stream) {
  if (!Q || !D) return LIK_ERR_INVALID;
  if (Q->dtype != D->dtype || Q->dim != D->dim || Q->dim <= 0) return LIK_ERR_INVALID;
  if (Q->dtype != LIK_BF16 && Q->dtype != LIK_F16 && Q->dtype != LIK_F32) return LIK_ERR_UNSUPPORTED;
  if (Q->lengths || Q->token_scale || D->token_scale) return LIK_ERR_UNSUPPORTED;
  // doc masks / lengths act through the forward's argmax; a packed side is
  // never normalised here (its row count is only known on the device)
  if ((Q->cu_seqlens && bwd_norm_q(flags)) || (D->cu_seqlens && bwd_norm_d(flags))) return LIK_ERR_UNSUPPORTED;
  if (D->cu_seqlens && (flags & LIK_KD_LAYOUT)) return LIK_ERR_INVALID;
  if (Q->n < 0 || D->n < 0 || Q->len < 0 || D->len < 0) return LIK_ERR_INVALID;
  if (Q->dim > 2048) return LIK_ERR_UNSUPPORTED;
  const bool kd = (flags & LIK_KD_LAYOUT) != 0;
  if (kd && (Q->n == 0 || D->n % Q->n != 0)) return LIK_ERR_INVALID;
  if (Q->n == 0 || D->n == 0) return LIK_OK;
  if (!grad || !argmax || !grad_q || !Q->data || !D->data) return LIK_ERR_INVALID;
  hipStream_t s = (hipStream_t)stream;
  const int eb = elem_size(Q->dtype);
  BwdParams bp{};
  bp.qsplit = 1;
  bp.grad = grad;
  bp.ld_g = grad_ld;
  bp.q = (const char*)Q->data;
  bp.q_sn = Q->stride_n * eb;
  bp.q_sl = Q->stride_l * eb;
  bp.q_cu = Q->cu_seqlens;
  bp.d = (const char*)D->data;
  bp.d_sn = D->stride_n * eb;
  bp.d_sl = D->stride_l * eb;
  bp.d_cu = D->cu_seqlens;
  bp.amax = argmax;
  bp.qmask = Q->mask;
  bp.qm_sn = Q->mask_stride_n;
  bp.qm_sl = Q->mask_stride_l;
  bp.gq = (char*)grad_q;
  bp.gd = (char*)grad_d;
  // 16-byte row chunks for the norm kernel
  if (((uintptr_t)Q->data) % 16 || ((uintptr_t)D->data) % 16 || (Q->dim * eb) % 16 || bp.q_sl % 16 || bp.d_sl % 16 ||
      bp.q_sn % 16 || bp.d_sn % 16)
    return LIK_ERR_UNSUPPORTED;
  bp.nq = Q->n;
  bp.lq = Q->len;
  bp.nd = D->n;
  bp.ld = D->len;
  bp.kd = kd ? 1 : 0;
  bp.ndoc_pg = kd ? D->n / Q->n : D->n;
  bp.dim = Q->dim;
  int rc;
  const size_t need = lik_maxsim_backward_workspace_size(Q, D, flags);
  if (need && (!workspace || workspace_bytes < need)) return LIK_ERR_WORKSPACE;
  float* wsf = (float*)workspace;
  auto invnorm = [&](const char* x, int64_t sn, int64_t sl, int64_t n, int64_t L, float* inv) {
    switch (Q->dtype) {
      case LIK_BF16: return launch_invnorm<EK_BF16>(x, sn, sl, n, L, Q->dim, inv, s);
      case LIK_F16: return launch_invnorm<EK_F16>(x, sn, sl, n, L, Q->dim, inv, s);
      default: return launch_invnorm<EK_F32>(x, sn, sl, n, L, Q->dim, inv, s);
    }
  };
  if (bwd_norm_q(flags)) {
    bp.qinv = wsf;
    wsf += Q->n * Q->len;
    if ((rc = invnorm(bp.q, bp.q_sn, bp.q_sl, Q->n, Q->len, wsf - Q->n * Q->len)) != LIK_OK) return rc;
  }
  if (bwd_norm_d(flags)) {
    bp.dinv = wsf;
    // fewer winner entries than doc rows (KD layout): norms of the winners only
    if (bp.amax && bp.nq * bp.ndoc_pg * bp.lq < D->n * D->len &&
        (bp.nq * bp.ndoc_pg * bp.lq) * 16 < ((int64_t)1 << 31) * 256) {
      switch (Q->dtype) {
        case LIK_BF16: rc = launch_winner_invnorm<EK_BF16>(bp, wsf, s); break;
        case LIK_F16: rc = launch_winner_invnorm<EK_F16>(bp, wsf, s); break;
        default: rc = launch_winner_invnorm<EK_F32>(bp, wsf, s); break;
      }
      if (rc != LIK_OK) return rc;
    } else if ((rc = invnorm(bp.d, bp.d_sn, bp.d_sl, D->n, D->len, wsf)) != LIK_OK) {
      return rc;
    }
  }
  char* wcur = (char*)workspace + align256(bwd_norm_floats(Q, D, flags) * sizeof(float));
  if (grad_q_part_bytes(Q, D, flags)) {
    int64_t split;
    grad_q_split(Q, D, flags, &split, &bp.qchunk);
    bp.qsplit = (int)split;
    bp.gq_part = (float*)wcur;
  }
  wcur += align256(grad_q_part_bytes(Q, D, flags));
  const RowWs rw = grad_d ? row_ws_layout(Q, D, flags) : RowWs{};
  if (rw.total) {
    char* ws = (char*)(((uintptr_t)wcur + 255) & ~(uintptr_t)255);
    auto I = [&](size_t off) { return (int32_t*)(ws + off); };
    hipLaunchKernelGGL(row_keys_kernel, dim3((unsigned)((rw.n + 255) / 256)), dim3(256), 0, s, bp, rw.n, I(rw.kin),
                       I(rw.vin));
    if (hipGetLastError() != hipSuccess) return LIK_ERR_LAUNCH;
    size_t tb = rw.temp_bytes;
    if (hipcub::DeviceRadixSort::SortPairs(ws + rw.temp, tb, I(rw.kin), I(rw.kout), I(rw.vin), I(rw.vout), (int)rw.n,
                                           0, end_bit_for(rw.rows), s) != hipSuccess)
      return LIK_ERR_LAUNCH;
    hipLaunchKernelGGL(bucket_ptr_kernel, dim3((unsigned)((rw.rows + 1 + 255) / 256)), dim3(256), 0, s, I(rw.kout),
                       rw.n, rw.rows, I(rw.ptr));
    if (hipGetLastError() != hipSuccess) return LIK_ERR_LAUNCH;
    bp.row_ptr = I(rw.ptr);
    bp.row_vals = I(rw.vout);
  }
  switch (Q->dtype) {
    case LIK_BF16: return launch_bwd_dpl<EK_BF16>(bp, s);
    case LIK_F16: return launch_bwd_dpl<EK_F16>(bp, s);
    default: return launch_bwd_dpl<EK_F32>(bp, s);
  }
}

int lik_maxsim_pairs_backward(const float* grad, const lik_seqs_t* Q, const lik_seqs_t* D, const int32_t* pair_q,
                              const int32_t* pair_d, int64_t num_pairs, const int32_t* argmax, uint32_t flags,
                              void* grad_q, void* grad_d, void* workspace, size_t workspace_bytes,
                              lik_stream_t stream) {
  if (!Q || !D || num_pairs < 0) return LIK_ERR_INVALID;
  if (Q->dtype != D->dtype || Q->dim != D->dim || Q->dim <= 0) return LIK_ERR_INVALID;
  if (Q->dtype != LIK_BF16 && Q->dtype != LIK_F16 && Q->dtype != LIK_F32) return LIK_ERR_UNSUPPORTED;
  if (Q->lengths || D->lengths || Q->token_scale || D->token_scale || D->mask) return LIK_ERR_UNSUPPORTED;
  if (flags & (LIK_NORMALIZE | LIK_NORMALIZE_Q | LIK_NORMALIZE_D | LIK_KD_LAYOUT)) return LIK_ERR_UNSUPPORTED;
  if (Q->dim > 2048) return LIK_ERR_UNSUPPORTED;
  if (Q->n < 0 || D->n < 0 || Q->len < 0 || D->len < 0) return LIK_ERR_INVALID;
  if (num_pairs > 0x7fffffffLL || Q->n > 0x7ffffffeLL || D->n > 0x7ffffffeLL) return LIK_ERR_UNSUPPORTED;
  if (num_pairs == 0 || Q->n == 0 || D->n == 0) return LIK_OK;
  if (!grad || !pair_q || !pair_d || !argmax || !grad_q || !Q->data || !D->data) return LIK_ERR_INVALID;
  const int eb = elem_size(Q->dtype);
  if (((uintptr_t)Q->data) % 16 || ((uintptr_t)D->data) % 16 || (Q->dim * eb) % 16 || (Q->stride_l * eb) % 16 ||
      (D->stride_l * eb) % 16 || (Q->stride_n * eb) % 16 || (D->stride_n * eb) % 16)
    return LIK_ERR_UNSUPPORTED;
  const PairWs w = pair_ws_layout(num_pairs, Q->n, D->n);
  if (!workspace || workspace_bytes < w.total) return LIK_ERR_WORKSPACE;
  char* ws = (char*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  if ((size_t)(ws - (char*)workspace) + w.total - 256 > workspace_bytes) return LIK_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  auto I = [&](size_t off) { return (int32_t*)(ws + off); };
  const unsigned pb = (unsigned)((num_pairs + 255) / 256);
  hipLaunchKernelGGL(pair_keys_kernel, dim3(pb), dim3(256), 0, s, pair_q, pair_d, num_pairs, Q->n, D->n, I(w.kq),
                     I(w.kd), I(w.iota));
  if (hipGetLastError() != hipSuccess) return LIK_ERR_LAUNCH;
  const int eb_bits = end_bit_for(Q->n > D->n ? Q->n : D->n);
  // stable LSD radix sort: pairs of one owner keep increasing pair order
  struct Pass { size_t key, list, ptr; int64_t n; } passes[2] = {{w.kq, w.qlist, w.qptr, Q->n},
                                                               {w.kd, w.dlist, w.dptr, D->n}};
  for (const Pass& ps : passes) {
    size_t tb = w.temp_bytes;
    if (hipcub::DeviceRadixSort::SortPairs(ws + w.temp, tb, I(ps.key), I(w.ks), I(w.iota), I(ps.list),
                                           (int)num_pairs, 0, eb_bits, s) != hipSuccess)
      return LIK_ERR_LAUNCH;
    hipLaunchKernelGGL(bucket_ptr_kernel, dim3((unsigned)((ps.n + 1 + 255) / 256)), dim3(256), 0, s, I(w.ks),
                       num_pairs, ps.n, I(ps.ptr));
    if (hipGetLastError() != hipSuccess) return LIK_ERR_LAUNCH;
  }
  BwdParams bp{};
  bp.qsplit = 1;
  bp.grad = grad;
  bp.ld_g = 1;
  bp.q = (const char*)Q->data;
  bp.q_sn = Q->stride_n * eb;
  bp.q_sl = Q->stride_l * eb;
  bp.q_cu = Q->cu_seqlens;
  bp.d = (const char*)D->data;
  bp.d_sn = D->stride_n * eb;
  bp.d_sl = D->stride_l * eb;
  bp.d_cu = D->cu_seqlens;
  bp.amax = argmax;
  bp.qmask = Q->mask;
  bp.qm_sn = Q->mask_stride_n;
  bp.qm_sl = Q->mask_stride_l;
  bp.gq = (char*)grad_q;
  bp.gd = (char*)grad_d;
  bp.nq = Q->n;
  bp.lq = Q->len;
  bp.nd = D->n;
  bp.ld = D->len;
  bp.kd = 0;
  bp.ndoc_pg = 0;
  bp.dim = Q->dim;
  bp.pair_q = pair_q;
  bp.pair_d = pair_d;
  bp.q_ptr = I(w.qptr);
  bp.q_list = I(w.qlist);
  bp.d_ptr = I(w.dptr);
  bp.d_list = I(w.dlist);
  switch (Q->dtype) {
    case LIK_BF16: return launch_bwd_dpl<EK_BF16>(bp, s);
    case LIK_F16: return launch_bwd_dpl<EK_F16>(bp, s);
    default: return launch_bwd_dpl<EK_F32>(bp, s);
  }
}

}  // extern "C"
