// MaxSim forward for gfx950: dense / KD / packed (varlen) / pair-list / fp8 /
// PLAID-residual documents, one kernel family.
//
// Work decomposition. A workgroup of W wavefronts owns a block of COLS =
// W*NSUB*32 query tokens ("columns"), held for the workgroup's lifetime in
// VGPRs as MFMA B-fragments, and walks a contiguous range of documents in
// 32-token tiles. Each tile is staged once through LDS (with the optional
// per-token L2 norm, mask bias and, for PLAID, the centroid+residual decode
// fused into the staging pass) and then multiplied by every wavefront
// against its own NSUB column blocks (v_mfma_f32_32x32x16_bf16/f16, or
// v_mfma_scale_f32_32x32x64_f8f6f4 for fp8). Doc tokens are the MFMA rows,
// so the max over doc tokens is an in-lane max over the 16 accumulator
// registers plus one lane^32 exchange at the end of a document; the
// [Nq, Nd, Lq, Ld] similarity tensor never exists, not even per tile in LDS.
// At a document's end the per-column maxima go through LDS and are summed
// per query in a fixed order (bitwise deterministic, no atomics).
//
// Semantics follow late_interaction_kernels/reference.py:26-98 (dense),
// 142-179 (residual), 213-245 (varlen), 248-269 (pairs): a doc-side mask
// removes tokens from the max, a query-side mask from the sum, a max over no
// valid token (or a non-finite max) contributes 0, normalise is
// x / max(||x||, 1e-12).
#include <math.h>

#include "lik_common.h"

namespace lik {

struct SeqDev {
  const char* data;
  int64_t sn_b, sl_b;  // byte strides
  const int32_t* cu;
  const int32_t* lengths;
  const int8_t* mask;
  int64_t msn, msl;
  const float* ts;
  int64_t tsn, tsl;
  int64_t n, L;
  int dim;
};

struct PlaidDev {
  const int32_t* codes;
  const uint8_t* res;
  const int32_t* cu;
  const int32_t* lengths;
  int64_t n, L, codes_sn, res_st;
  const char* cent;
  int64_t cent_sb;
  int64_t ncent;
  const float* bw;
  int nb, nbits;
};

struct Params {
  SeqDev q;
  SeqDev d;
  PlaidDev pl;
  const int32_t* extent;  // per-doc valid extent from the mask pre-pass
  const uint8_t* holes;   // per-doc: mask has a False inside [0, extent)
  const int32_t* pair_q;
  const int32_t* pair_d;
  int64_t nunits;  // query units (query x Lq-chunk); pair mode: number of pairs
  int nc;          // Lq chunks per query
  int LU;          // columns per unit
  int QPG;         // units per column group
  int64_t ngroups;
  int64_t ndocs_pg;  // docs per group
  int64_t kd_K;      // KD layout: docs per query (0: cross product)
  int R;             // docs per workgroup
  int64_t NR;        // doc ranges per group
  int xcd_map;
  int normalize;
  float out_scale;
  float* out;
  int64_t osq, osd;
};

enum { SRC_DENSE = 0, SRC_PLAID = 1 };

__device__ __forceinline__ int64_t seq_len(const SeqDev& s, int64_t i) {
  if (s.cu) return (int64_t)s.cu[i + 1] - s.cu[i];
  if (s.lengths) {
    const int64_t l = s.lengths[i];
    return l < 0 ? 0 : (l > s.L ? s.L : l);
  }
  return s.L;
}
__device__ __forceinline__ const char* seq_row0(const SeqDev& s, int64_t i) {
  return s.cu ? s.data + (int64_t)s.cu[i] * s.sl_b : s.data + i * s.sn_b;
}

template <int SRC>
__device__ __forceinline__ int64_t doc_len(const Params& p, int64_t j) {
  if (j < 0) return 0;  // out-of-range pair index scores 0
  if constexpr (SRC == SRC_PLAID) {
    if (p.pl.cu) return (int64_t)p.pl.cu[j + 1] - p.pl.cu[j];
    const int64_t l = p.pl.lengths[j];
    return l < 0 ? 0 : (l > p.pl.L ? p.pl.L : l);
  } else {
    if (p.extent) return p.extent[j];
    return seq_len(p.d, j);
  }
}

// Config legality: B-fragment registers per lane must stay <= 128 VGPRs.
template <int EK, int DPAD, int NSUB>
constexpr bool cfg_ok() {
  using T = KT<EK, DPAD>;
  return T::KSTEPS >= 1 && T::CPR <= 64 &&
         NSUB * T::KSTEPS * T::FRAG_V * 4 * (T::SPLIT ? 2 : 1) <= 128;
}

template <int EK, int DPAD, int W, int NSUB, int SRC, int CD>
__global__ void __launch_bounds__(W * 64) maxsim_kernel(const Params p) {
  using T = KT<EK, DPAD>;
  constexpr int NT = W * 64;
  constexpr int COLS = W * NSUB * 32;
  constexpr int KS = T::KSTEPS;
  constexpr int FV = T::FRAG_V;
  // 16-byte staging chunks per row: input chunks (dense) or output chunks of 8 dims (PLAID)
  constexpr int SCPR = SRC == SRC_DENSE ? T::CPR : DPAD / 8;
  constexpr int NCH = (32 * SCPR + NT - 1) / NT;
  constexpr float NEG_INF = -__builtin_huge_valf();
  static_assert(SRC == SRC_DENSE || !T::SPLIT, "PLAID computes in bf16/f16");
  static_assert(SRC == SRC_DENSE || EK != EK_FP8, "PLAID computes in bf16/f16");

  __shared__ __attribute__((aligned(16))) char s_tile[2][T::NARR][T::TILE_B];
  __shared__ __attribute__((aligned(16))) float s_rs[2][32];
  __shared__ __attribute__((aligned(16))) float s_rb[2][32];
  __shared__ float s_col[COLS];
  __shared__ float s_bw[SRC == SRC_PLAID ? 256 : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wv = tid >> 6, h = lane >> 5, l32 = lane & 31;

  int64_t g, r;
  {
    const int64_t b = blockIdx.x;
    if (p.xcd_map) {
      // Dispatch is round-robin over the 8 XCDs: give every XCD whole doc
      // ranges, with all column groups of one range landing on the same XCD
      // back to back, so the range's tiles are fetched into that XCD's L2 once.
      const int64_t i = b >> 3;
      g = i % p.ngroups;
      r = (i / p.ngroups) * 8 + (b & 7);
    } else {
      g = b % p.ngroups;
      r = b / p.ngroups;
    }
  }
  if (r >= p.NR) return;

  if constexpr (SRC == SRC_PLAID) {
    for (int i = tid; i < 256; i += NT) s_bw[i] = i < p.pl.nb ? p.pl.bw[i] : 0.f;
  }

  // ---------------- query block -> B fragments in VGPRs ----------------
  u32x4 bq[NSUB][KS][FV];
  u32x4 bql[T::SPLIT ? NSUB : 1][T::SPLIT ? KS : 1];
  float qsc[NSUB];
#pragma unroll
  for (int sub = 0; sub < NSUB; ++sub) {
    const int col = (wv * NSUB + sub) * 32 + l32;
    const int ul = col / p.LU;
    const int s = col - ul * p.LU;
    bool valid = ul < p.QPG;
    int64_t q = 0, tok = 0;
    if (p.pair_q) {
      q = p.pair_q[g];
      tok = s;
      valid = valid && q >= 0 && q < p.q.n;
    } else {
      const int64_t u = g * p.QPG + ul;
      valid = valid && u < p.nunits;
      q = u / p.nc;
      tok = (u - q * p.nc) * (int64_t)p.LU + s;
    }
    const char* rowp = nullptr;
    if (valid) {
      valid = tok < seq_len(p.q, q);
      if (valid && p.q.mask) valid = p.q.mask[q * p.q.msn + tok * p.q.msl] != 0;
      rowp = seq_row0(p.q, q) + tok * p.q.sl_b;
    }
    float ss = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      constexpr int NIN = T::FE * T::IN_B / 16;  // 16-B input chunks per fragment
      u32x4 raw[NIN];
#pragma unroll
      for (int c = 0; c < NIN; ++c) {
        const int e = h * (DPAD / 2) + ks * T::FE + c * T::CHUNK_E;
        raw[c] = (valid && e < p.q.dim) ? *(const u32x4*)(rowp + (int64_t)e * T::IN_B)
                                        : (u32x4){0u, 0u, 0u, 0u};
        if (p.normalize) ss += chunk_sumsq<EK>(raw[c]);
      }
      if constexpr (T::SPLIT) {
        u32x2 h0, l0, h1, l1;
        split4(raw[0], h0, l0);
        split4(raw[NIN > 1 ? 1 : 0], h1, l1);
        bq[sub][ks][0] = (u32x4){h0[0], h0[1], h1[0], h1[1]};
        bql[sub][ks] = (u32x4){l0[0], l0[1], l1[0], l1[1]};
      } else {
#pragma unroll
        for (int c = 0; c < FV; ++c) bq[sub][ks][c] = raw[c];
      }
    }
    ss += __shfl_xor(ss, 32);
    float sc = p.normalize ? inv_norm(ss) : 1.f;
    if (valid && p.q.ts) sc *= p.q.ts[q * p.q.tsn + tok * p.q.tsl];
    qsc[sub] = valid ? sc : 0.f;
  }

  // ---------------- document range ----------------
  const int64_t jl0 = r * (int64_t)p.R;
  const int64_t jl1 = (jl0 + p.R < p.ndocs_pg) ? jl0 + p.R : p.ndocs_pg;
  const int64_t kd_base = p.kd_K ? (g / p.nc) * p.kd_K : 0;  // KD: QPG == 1
  auto dglob = [&](int64_t jl) -> int64_t {
    if (p.pair_d) {
      const int64_t pd = p.pair_d[g];
      return (pd >= 0 && pd < p.d.n) ? pd : -1;
    }
    return kd_base + jl;
  };
  auto unit_of = [&](int t) -> int64_t { return p.pair_q ? g : g * p.QPG + t; };

  for (int64_t jl = jl0; jl < jl1; ++jl) {
    if (doc_len<SRC>(p, dglob(jl)) == 0) {
      for (int t = tid; t < p.QPG; t += NT) {
        const int64_t u = unit_of(t);
        if (u < p.nunits) p.out[u * p.osq + jl * p.osd] = 0.f;
      }
    }
  }
  auto first_from = [&](int64_t jl) -> int64_t {
    while (jl < jl1 && doc_len<SRC>(p, dglob(jl)) == 0) ++jl;
    return jl;
  };

  int64_t cj = first_from(jl0);
  if (cj >= jl1) return;
  int64_t cdoc = dglob(cj);
  int64_t clen = doc_len<SRC>(p, cdoc);
  int ct = 0;

  // ---- staging registers (the next tile, loaded while the current one computes)
  u32x4 st[NCH];
  u32x4 st2[SRC == SRC_PLAID && CD == EK_F32 ? NCH : 1];  // second half of fp32 centroid chunk
  uint64_t stbits[SRC == SRC_PLAID ? NCH : 1];
  bool stok[NCH];
  float stts[NCH];

  auto prefetch = [&](int64_t doc, int64_t len, int t) {
    if constexpr (SRC == SRC_DENSE) {
      const char* base = seq_row0(p.d, doc);
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const int c = tid + i * NT;
        const int row = c / SCPR, cc = c % SCPR;
        const int64_t tok = (int64_t)t * 32 + row;
        const bool inr = c < 32 * SCPR && tok < len;
        const bool ld = inr && cc * T::CHUNK_E < p.d.dim;
        st[i] = ld ? *(const u32x4*)(base + tok * p.d.sl_b + cc * 16) : (u32x4){0u, 0u, 0u, 0u};
        bool ok = inr;
        float ts = 1.f;
        if (cc == 0 && inr) {
          if (p.d.mask) ok = p.d.mask[doc * p.d.msn + tok * p.d.msl] != 0;
          if (p.d.ts) ts = p.d.ts[doc * p.d.tsn + tok * p.d.tsl];
        }
        stok[i] = ok;
        stts[i] = ts;
      }
    } else {
      const int64_t tok0 = p.pl.cu ? (int64_t)p.pl.cu[doc] : doc * p.pl.codes_sn;
      constexpr int CSZ = CD == EK_F32 ? 4 : 2;
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const int c = tid + i * NT;
        const int row = c / SCPR, cc = c % SCPR;
        const int64_t tl = (int64_t)t * 32 + row;
        const bool inr = c < 32 * SCPR && tl < len;
        const bool ld = inr && cc * 8 < p.q.dim;
        u32x4 a = {0u, 0u, 0u, 0u}, b = {0u, 0u, 0u, 0u};
        uint64_t bits = 0;
        if (ld) {
          const int64_t tk = tok0 + tl;
          int64_t code = p.pl.codes[tk];
          code = (code < 0 || code >= p.pl.ncent) ? 0 : code;
          const char* cp = p.pl.cent + code * p.pl.cent_sb + (int64_t)cc * 8 * CSZ;
          a = *(const u32x4*)cp;
          if constexpr (CD == EK_F32) b = *(const u32x4*)(cp + 16);
          const uint8_t* rp = p.pl.res + tk * p.pl.res_st + (int64_t)cc * p.pl.nbits;
          if (p.pl.nbits == 2) bits = *(const uint16_t*)rp;
          else if (p.pl.nbits == 4) bits = *(const uint32_t*)rp;
          else bits = *(const uint64_t*)rp;
        }
        st[i] = a;
        if constexpr (CD == EK_F32) st2[i] = b;
        stbits[i] = bits;
        stok[i] = inr;
        stts[i] = 1.f;
      }
    }
  };

  auto commit = [&](int buf) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = tid + i * NT;
      const int row = c / SCPR, cc = c % SCPR;
      const bool inr = c < 32 * SCPR;
      if constexpr (SRC == SRC_DENSE) {
        float ss = 0.f;
        if (p.normalize) {
          ss = chunk_sumsq<EK>(st[i]);
#pragma unroll
          for (int o = 1; o < SCPR; o <<= 1) ss += __shfl_xor(ss, o);
        }
        if (inr) {
          char* rowp = s_tile[buf][0] + row * T::ROW_B;
          if constexpr (T::SPLIT) {
            u32x2 hi, lo;
            split4(st[i], hi, lo);
            *(u32x2*)(rowp + cc * 8) = hi;
            *(u32x2*)(s_tile[buf][1] + row * T::ROW_B + cc * 8) = lo;
          } else {
            *(u32x4*)(rowp + cc * 16) = st[i];
          }
          if (cc == 0) {
            s_rs[buf][row] = (p.normalize ? inv_norm(ss) : 1.f) * stts[i];
            s_rb[buf][row] = stok[i] ? 0.f : NEG_INF;
          }
        }
      } else {
        // decode 8 dims: centroid + bucket weight
        float x[8];
        const uint32_t bmask = (1u << p.pl.nbits) - 1u;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float cv;
          if constexpr (CD == EK_F32) cv = __uint_as_float(e < 4 ? st[i][e] : st2[i][e - 4]);
          else if constexpr (CD == EK_BF16)
            cv = (e & 1) ? bf16hi_to_f32(st[i][e >> 1]) : bf16lo_to_f32(st[i][e >> 1]);
          else cv = f16_to_f32((uint16_t)((e & 1) ? (st[i][e >> 1] >> 16) : (st[i][e >> 1] & 0xffffu)));
          uint32_t bc = (uint32_t)(stbits[i] >> (e * p.pl.nbits)) & bmask;
          bc = bc < (uint32_t)p.pl.nb ? bc : (uint32_t)(p.pl.nb - 1);
          const bool live = stok[i] && (cc * 8 + e) < p.q.dim;
          x[e] = live ? cv + s_bw[bc] : 0.f;
        }
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
#pragma unroll
        for (int o = 1; o < SCPR; o <<= 1) ss += __shfl_xor(ss, o);
        const float sc = p.normalize ? inv_norm(ss) : 1.f;
        if (inr) {
          u32x4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if constexpr (EK == EK_F16)
              w[e] = f32_to_f16_bits(x[2 * e] * sc) | (f32_to_f16_bits(x[2 * e + 1] * sc) << 16);
            else
              w[e] = f32_to_bf16_bits(x[2 * e] * sc) | (f32_to_bf16_bits(x[2 * e + 1] * sc) << 16);
          }
          *(u32x4*)(s_tile[buf][0] + row * T::ROW_B + cc * 16) = w;
          if (cc == 0) {
            s_rs[buf][row] = 1.f;
            s_rb[buf][row] = stok[i] ? 0.f : NEG_INF;
          }
        }
      }
    }
  };

  float m[NSUB];
#pragma unroll
  for (int sub = 0; sub < NSUB; ++sub) m[sub] = NEG_INF;

  const bool dense_fix = SRC == SRC_DENSE && (p.normalize || p.d.ts != nullptr);
  int buf = 0;
  prefetch(cdoc, clen, 0);
  while (true) {
    commit(buf);
    __syncthreads();

    int64_t nj = cj, ndoc = cdoc, nlen = clen;
    int nt = ct + 1;
    if ((int64_t)nt * 32 >= clen) {
      nj = first_from(cj + 1);
      nt = 0;
      if (nj < jl1) {
        ndoc = dglob(nj);
        nlen = doc_len<SRC>(p, ndoc);
      }
    }
    const bool has_next = nj < jl1;
    if (has_next) prefetch(ndoc, nlen, nt);

    // ---- MFMA over the staged tile
    f32x16 acc[NSUB];
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[sub][e] = 0.f;
    const char* A = s_tile[buf][0] + l32 * T::ROW_B + h * T::HALF_B;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 a[FV];
#pragma unroll
      for (int v = 0; v < FV; ++v) a[v] = *(const u32x4*)(A + ks * T::FRAG_B + v * 16);
      if constexpr (T::SPLIT) {
        const u32x4 al = *(const u32x4*)(s_tile[buf][1] + l32 * T::ROW_B + h * T::HALF_B + ks * T::FRAG_B);
#pragma unroll
        for (int sub = 0; sub < NSUB; ++sub) {
          mfma32<EK>(acc[sub], a, bq[sub][ks]);
          mfma32<EK>(acc[sub], a, &bql[sub][ks]);
          mfma32<EK>(acc[sub], &al, bq[sub][ks]);
        }
      } else {
#pragma unroll
        for (int sub = 0; sub < NSUB; ++sub) mfma32<EK>(acc[sub], a, bq[sub][ks]);
      }
    }

    // ---- epilogue: running max over doc tokens (rows)
    const bool partial = (int64_t)(ct + 1) * 32 > clen;
    const bool fix = dense_fix || partial || (p.holes != nullptr && p.holes[cdoc] != 0);
    if (fix) {
      f32x4 sc[4], bi[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sc[j] = *(const f32x4*)&s_rs[buf][8 * j + 4 * h];
        bi[j] = *(const f32x4*)&s_rb[buf][8 * j + 4 * h];
      }
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) m[sub] = fmaxf(m[sub], fmaf(acc[sub][4 * j + e], sc[j][e], bi[j][e]));
    } else {
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
        for (int e = 0; e < 16; ++e) m[sub] = fmaxf(m[sub], acc[sub][e]);
    }

    // ---- end of document: per-column max -> per-unit sum
    if ((int64_t)(ct + 1) * 32 >= clen) {
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub) {
        const float mm = fmaxf(m[sub], __shfl_xor(m[sub], 32));
        const float v = __builtin_isfinite(mm) ? mm * qsc[sub] : 0.f;
        if (h == 0) s_col[(wv * NSUB + sub) * 32 + l32] = v;
        m[sub] = NEG_INF;
      }
      __syncthreads();
      for (int t = tid; t < p.QPG; t += NT) {
        const int64_t u = unit_of(t);
        if (u < p.nunits) {
          const float* cv = s_col + t * p.LU;
          int k = t % p.LU;  // rotated start: spreads LDS banks across threads
          float sum = 0.f;
          for (int s = 0; s < p.LU; ++s) {
            sum += cv[k];
            k = (k + 1 == p.LU) ? 0 : k + 1;
          }
          p.out[u * p.osq + cj * p.osd] = sum * p.out_scale;
        }
      }
    }

    if (!has_next) break;
    cj = nj;
    ct = nt;
    cdoc = ndoc;
    clen = nlen;
    buf ^= 1;
  }
}

// Per-document valid extent of a boolean mask: extent = last kept token + 1,
// holes = some token inside [0, extent) is dropped. One wavefront per doc.
__global__ void __launch_bounds__(256) doc_extent_kernel(const int8_t* mask, int64_t msn, int64_t msl,
                                                         int64_t n, int64_t L, const int32_t* lengths,
                                                         int32_t* extent, uint8_t* holes) {
  const int64_t j = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (j >= n) return;
  int64_t Lj = L;
  if (lengths) {
    const int64_t l = lengths[j];
    Lj = l < 0 ? 0 : (l > L ? L : l);
  }
  int last = -1, cnt = 0;
  for (int64_t t = lane; t < Lj; t += 64) {
    if (mask[j * msn + t * msl] != 0) {
      last = (int)t;
      ++cnt;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    last = max(last, __shfl_xor(last, o));
    cnt += __shfl_xor(cnt, o);
  }
  if (lane == 0) {
    extent[j] = last + 1;
    holes[j] = (uint8_t)(cnt != last + 1);
  }
}

// out[q, j] = sum_c part[q*nc + c, j], c ascending.
__global__ void __launch_bounds__(256) unit_sum_kernel(const float* part, int64_t nq, int nc, int64_t nd,
                                                       float* out, int64_t osq, int64_t osd) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nq * nd) return;
  const int64_t q = i / nd, j = i - q * nd;
  float s = 0.f;
  for (int c = 0; c < nc; ++c) s += part[(q * nc + c) * nd + j];
  out[q * osq + j * osd] = s;
}

}  // namespace lik

// ============================================================================
// Host side: validation, configuration and launch.
// ============================================================================
using namespace lik;

namespace {

struct Cfg {
  int W, NSUB;
};
// Column-block configurations, smallest first.
constexpr Cfg kCfgs[] = {{1, 1}, {1, 2}, {1, 4}, {4, 1}, {4, 2}, {4, 4}};
constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

int elem_bytes(int dt) { return dt == LIK_F32 ? 4 : (dt == LIK_FP8_E4M3 ? 1 : 2); }

int pick_dpad(int dt, int dim) {
  const int opts[] = {64, 128, 256, 512};
  for (int o : opts)
    if (dim <= o) {
      if (dt == LIK_F32 && o > 256) return -1;
      if (dt == LIK_FP8_E4M3 && o > 256) return -1;
      return o;
    }
  return -1;
}

int max_nsub(int dt, int dpad) {
  const int fe = dt == LIK_FP8_E4M3 ? 32 : 8;
  const int cb = dt == LIK_FP8_E4M3 ? 1 : 2;
  const int ks = dpad / (2 * fe);
  const int fv = fe * cb / 16;
  const int per = ks * fv * 4 * (dt == LIK_F32 ? 2 : 1);
  int n = 128 / per;
  return n > 4 ? 4 : n;
}

SeqDev to_dev(const lik_seqs_t& s) {
  SeqDev d;
  const int eb = elem_bytes(s.dtype);
  d.data = (const char*)s.data;
  d.sn_b = s.stride_n * eb;
  d.sl_b = s.stride_l * eb;
  d.cu = s.cu_seqlens;
  d.lengths = s.lengths;
  d.mask = s.mask;
  d.msn = s.mask_stride_n;
  d.msl = s.mask_stride_l;
  d.ts = s.token_scale;
  d.tsn = s.scale_stride_n;
  d.tsl = s.scale_stride_l;
  d.n = s.n;
  d.L = s.len;
  d.dim = s.dim;
  return d;
}

int check_seqs(const lik_seqs_t* s) {
  if (!s || s->n < 0 || s->len < 0 || s->dim <= 0) return LIK_ERR_INVALID;
  if (s->dtype < LIK_BF16 || s->dtype > LIK_FP8_E4M3) return LIK_ERR_INVALID;
  if (s->n > 0 && s->len > 0 && !s->data) return LIK_ERR_INVALID;
  const int eb = elem_bytes(s->dtype);
  if ((s->dim * eb) % 16 != 0) return LIK_ERR_UNSUPPORTED;
  if (((uintptr_t)s->data) % 16 != 0) return LIK_ERR_UNSUPPORTED;
  if ((s->stride_l * eb) % 16 != 0) return LIK_ERR_UNSUPPORTED;
  if (!s->cu_seqlens && (s->stride_n * eb) % 16 != 0) return LIK_ERR_UNSUPPORTED;
  if (s->cu_seqlens && (s->mask || s->lengths)) return LIK_ERR_INVALID;
  if (s->token_scale && s->dtype != LIK_FP8_E4M3) return LIK_ERR_INVALID;
  return LIK_OK;
}

struct Plan {
  int W = 0, NSUB = 0, dpad = 0;
  int LU = 0, QPG = 0, nc = 1;
  int64_t nunits = 0, ngroups = 0;
};

// Choose the column block, Lq chunking and grouping for `nq` queries of
// (max) length `lq`. `one_query_per_group` is true when each query owns its
// documents (KD / pairs).
int make_plan(int dt, int dim, int64_t nq, int64_t lq, bool one_query_per_group, Plan& pl) {
  pl.dpad = pick_dpad(dt, dim);
  if (pl.dpad < 0) return LIK_ERR_UNSUPPORTED;
  const int nsmax = max_nsub(dt, pl.dpad);
  if (lq < 1) lq = 1;
  const int64_t need = one_query_per_group ? lq : nq * lq;
  int best = -1;
  for (int i = 0; i < kNumCfgs; ++i) {
    if (kCfgs[i].NSUB > nsmax) continue;
    best = i;
    if ((int64_t)kCfgs[i].W * kCfgs[i].NSUB * 32 >= need) break;
  }
  if (best < 0) return LIK_ERR_UNSUPPORTED;
  pl.W = kCfgs[best].W;
  pl.NSUB = kCfgs[best].NSUB;
  const int cols = pl.W * pl.NSUB * 32;
  if (lq <= cols) {
    pl.nc = 1;
    pl.LU = (int)lq;
    pl.QPG = one_query_per_group ? 1 : cols / (int)lq;
  } else {
    // Split each query into nc chunks; pick the chunking that wastes the
    // fewest columns (MaxSim is a sum over query tokens, so chunks add up).
    double best_eff = -1.0;
    for (int nc = (int)((lq + cols - 1) / cols); nc <= (int)((lq + cols - 1) / cols) + 8; ++nc) {
      const int lu = (int)((lq + nc - 1) / nc);
      const int qpg = one_query_per_group ? 1 : cols / lu;
      const double eff = (double)qpg * lu / cols;
      if (eff > best_eff + 1e-9) {
        best_eff = eff;
        pl.nc = nc;
        pl.LU = lu;
        pl.QPG = qpg;
      }
      if (one_query_per_group) break;
    }
  }
  pl.nunits = nq * pl.nc;
  pl.ngroups = one_query_per_group ? pl.nunits : (pl.nunits + pl.QPG - 1) / pl.QPG;
  return LIK_OK;
}

// Docs per workgroup: aim for >= ~2048 workgroups so 256 CUs see several
// waves of work, but keep at least a few docs per workgroup to amortise the
// query-block load.
int pick_R(int64_t ngroups, int64_t ndocs) {
  const int64_t target = 2048;
  int64_t R = (ndocs * ngroups) / target;
  if (R < 1) R = 1;
  if (R > ndocs) R = ndocs > 0 ? ndocs : 1;
  if (R > (1 << 20)) R = 1 << 20;
  return (int)R;
}

template <int EK, int DPAD, int W, int NSUB, int SRC, int CD>
int launch_one(const Params& p, int64_t nblocks, hipStream_t s) {
  if constexpr (!cfg_ok<EK, DPAD, NSUB>()) {
    return LIK_ERR_UNSUPPORTED;
  } else {
    if (nblocks <= 0) return LIK_OK;
    if (nblocks > 0x7fffffffLL) return LIK_ERR_UNSUPPORTED;
    hipLaunchKernelGGL((maxsim_kernel<EK, DPAD, W, NSUB, SRC, CD>), dim3((unsigned)nblocks),
                       dim3(W * 64), 0, s, p);
    return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
  }
}

template <int EK, int DPAD, int SRC, int CD>
int launch_cfg(const Plan& pl, const Params& p, int64_t nb, hipStream_t s) {
  if (pl.W == 1 && pl.NSUB == 1) return launch_one<EK, DPAD, 1, 1, SRC, CD>(p, nb, s);
  if (pl.W == 1 && pl.NSUB == 2) return launch_one<EK, DPAD, 1, 2, SRC, CD>(p, nb, s);
  if (pl.W == 1 && pl.NSUB == 4) return launch_one<EK, DPAD, 1, 4, SRC, CD>(p, nb, s);
  if (pl.W == 4 && pl.NSUB == 1) return launch_one<EK, DPAD, 4, 1, SRC, CD>(p, nb, s);
  if (pl.W == 4 && pl.NSUB == 2) return launch_one<EK, DPAD, 4, 2, SRC, CD>(p, nb, s);
  if (pl.W == 4 && pl.NSUB == 4) return launch_one<EK, DPAD, 4, 4, SRC, CD>(p, nb, s);
  return LIK_ERR_UNSUPPORTED;
}

template <int EK, int SRC, int CD>
int launch_dpad(const Plan& pl, const Params& p, int64_t nb, hipStream_t s) {
  switch (pl.dpad) {
    case 64: return launch_cfg<EK, 64, SRC, CD>(pl, p, nb, s);
    case 128: return launch_cfg<EK, 128, SRC, CD>(pl, p, nb, s);
    case 256: return launch_cfg<EK, 256, SRC, CD>(pl, p, nb, s);
    case 512:
      if constexpr (EK == EK_BF16 || EK == EK_F16) return launch_cfg<EK, 512, SRC, CD>(pl, p, nb, s);
      else return LIK_ERR_UNSUPPORTED;
    default: return LIK_ERR_UNSUPPORTED;
  }
}

int launch_dense(int dt, const Plan& pl, const Params& p, int64_t nb, hipStream_t s) {
  switch (dt) {
    case LIK_BF16: return launch_dpad<EK_BF16, SRC_DENSE, 0>(pl, p, nb, s);
    case LIK_F16: return launch_dpad<EK_F16, SRC_DENSE, 0>(pl, p, nb, s);
    case LIK_F32: return launch_dpad<EK_F32, SRC_DENSE, 0>(pl, p, nb, s);
    case LIK_FP8_E4M3: return launch_dpad<EK_FP8, SRC_DENSE, 0>(pl, p, nb, s);
    default: return LIK_ERR_UNSUPPORTED;
  }
}

template <int EK, int CD>
int launch_plaid_dpad(const Plan& pl, const Params& p, int64_t nb, hipStream_t s) {
  switch (pl.dpad) {
    case 64: return launch_cfg<EK, 64, SRC_PLAID, CD>(pl, p, nb, s);
    case 128: return launch_cfg<EK, 128, SRC_PLAID, CD>(pl, p, nb, s);
    case 256: return launch_cfg<EK, 256, SRC_PLAID, CD>(pl, p, nb, s);
    default: return LIK_ERR_UNSUPPORTED;
  }
}

int launch_plaid(int dt, int cd, const Plan& pl, const Params& p, int64_t nb, hipStream_t s) {
  if (dt == LIK_BF16) {
    if (cd == LIK_BF16) return launch_plaid_dpad<EK_BF16, EK_BF16>(pl, p, nb, s);
    if (cd == LIK_F16) return launch_plaid_dpad<EK_BF16, EK_F16>(pl, p, nb, s);
    if (cd == LIK_F32) return launch_plaid_dpad<EK_BF16, EK_F32>(pl, p, nb, s);
  } else if (dt == LIK_F16) {
    if (cd == LIK_BF16) return launch_plaid_dpad<EK_F16, EK_BF16>(pl, p, nb, s);
    if (cd == LIK_F16) return launch_plaid_dpad<EK_F16, EK_F16>(pl, p, nb, s);
    if (cd == LIK_F32) return launch_plaid_dpad<EK_F16, EK_F32>(pl, p, nb, s);
  }
  return LIK_ERR_UNSUPPORTED;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct WsLayout {
  size_t extent_off = 0, holes_off = 0, part_off = 0, total = 0;
  bool need_extent = false, need_part = false;
};

WsLayout ws_layout(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags, const Plan& pl) {
  WsLayout w;
  size_t off = 0;
  if (D->mask) {
    w.need_extent = true;
    w.extent_off = off;
    off = align256(off + sizeof(int32_t) * (size_t)D->n);
    w.holes_off = off;
    off = align256(off + (size_t)D->n);
  }
  if (pl.nc > 1) {
    const bool kd = (flags & LIK_KD_LAYOUT) != 0;
    const int64_t ndpg = kd ? (Q->n > 0 ? D->n / Q->n : 0) : D->n;
    w.need_part = true;
    w.part_off = off;
    off = align256(off + sizeof(float) * (size_t)(pl.nunits * ndpg));
  }
  w.total = off;
  return w;
}

}  // namespace

extern "C" {

const char* lik_version(void) { return "lik-hip 0.1.0 gfx950"; }

size_t lik_maxsim_workspace_size(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags) {
  if (check_seqs(Q) != LIK_OK || check_seqs(D) != LIK_OK) return 0;
  Plan pl;
  const bool kd = (flags & LIK_KD_LAYOUT) != 0;
  if (make_plan(Q->dtype, Q->dim, Q->n, Q->len, kd, pl) != LIK_OK) return 0;
  return ws_layout(Q, D, flags, pl).total;
}

int lik_maxsim(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags, float out_scale, float* out,
               int64_t out_stride_q, int64_t out_stride_d, void* workspace, size_t workspace_bytes,
               lik_stream_t stream) {
  int rc;
  if ((rc = check_seqs(Q)) != LIK_OK) return rc;
  if ((rc = check_seqs(D)) != LIK_OK) return rc;
  if (Q->dtype != D->dtype || Q->dim != D->dim) return LIK_ERR_INVALID;
  if (!out && Q->n > 0 && D->n > 0) return LIK_ERR_INVALID;
  const bool kd = (flags & LIK_KD_LAYOUT) != 0;
  if (kd && (D->cu_seqlens || (Q->n > 0 && D->n % Q->n != 0))) return LIK_ERR_INVALID;
  if (Q->n == 0 || D->n == 0) return LIK_OK;
  hipStream_t s = (hipStream_t)stream;

  Plan pl;
  if ((rc = make_plan(Q->dtype, Q->dim, Q->n, Q->len, kd, pl)) != LIK_OK) return rc;
  const WsLayout wl = ws_layout(Q, D, flags, pl);
  if (wl.total > 0 && (!workspace || workspace_bytes < wl.total)) return LIK_ERR_WORKSPACE;

  Params p{};
  p.q = to_dev(*Q);
  p.d = to_dev(*D);
  p.normalize = (flags & LIK_NORMALIZE) ? 1 : 0;
  p.out_scale = out_scale;
  p.nunits = pl.nunits;
  p.nc = pl.nc;
  p.LU = pl.LU;
  p.QPG = pl.QPG;
  p.ngroups = pl.ngroups;
  p.kd_K = kd ? D->n / Q->n : 0;
  p.ndocs_pg = kd ? p.kd_K : D->n;

  char* ws = (char*)workspace;
  if (wl.need_extent) {
    p.extent = (const int32_t*)(ws + wl.extent_off);
    p.holes = (const uint8_t*)(ws + wl.holes_off);
    hipLaunchKernelGGL(doc_extent_kernel, dim3((unsigned)((D->n + 3) / 4)), dim3(256), 0, s, D->mask,
                       D->mask_stride_n, D->mask_stride_l, D->n, D->len, D->lengths,
                       (int32_t*)(ws + wl.extent_off), (uint8_t*)(ws + wl.holes_off));
    if (hipGetLastError() != hipSuccess) return LIK_ERR_LAUNCH;
  }
  if (wl.need_part) {
    p.out = (float*)(ws + wl.part_off);
    p.osq = p.ndocs_pg;
    p.osd = 1;
  } else {
    p.out = out;
    p.osq = out_stride_q;
    p.osd = out_stride_d;
  }
  p.R = pick_R(p.ngroups, p.ndocs_pg);
  p.NR = (p.ndocs_pg + p.R - 1) / p.R;
  p.xcd_map = p.NR >= 8 ? 1 : 0;
  const int64_t nb = p.xcd_map ? p.ngroups * ((p.NR + 7) / 8) * 8 : p.ngroups * p.NR;
  if ((rc = launch_dense(Q->dtype, pl, p, nb, s)) != LIK_OK) return rc;
  if (wl.need_part) {
    const int64_t tot = Q->n * p.ndocs_pg;
    hipLaunchKernelGGL(unit_sum_kernel, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s,
                       (const float*)(ws + wl.part_off), Q->n, pl.nc, p.ndocs_pg, out, out_stride_q,
                       out_stride_d);
    if (hipGetLastError() != hipSuccess) return LIK_ERR_LAUNCH;
  }
  return LIK_OK;
}

int lik_maxsim_pairs(const lik_seqs_t* Q, const lik_seqs_t* D, const int32_t* pair_q, const int32_t* pair_d,
                     int64_t num_pairs, uint32_t flags, float* out, lik_stream_t stream) {
  int rc;
  if ((rc = check_seqs(Q)) != LIK_OK) return rc;
  if ((rc = check_seqs(D)) != LIK_OK) return rc;
  if (Q->dtype != D->dtype || Q->dim != D->dim) return LIK_ERR_INVALID;
  if (num_pairs < 0 || (num_pairs > 0 && (!pair_q || !pair_d || !out))) return LIK_ERR_INVALID;
  if (D->mask || (flags & LIK_KD_LAYOUT)) return LIK_ERR_INVALID;
  if (num_pairs == 0) return LIK_OK;
  Plan pl;
  if ((rc = make_plan(Q->dtype, Q->dim, 1, Q->len, true, pl)) != LIK_OK) return rc;
  if (pl.nc != 1) return LIK_ERR_UNSUPPORTED;
  Params p{};
  p.q = to_dev(*Q);
  p.d = to_dev(*D);
  p.normalize = (flags & LIK_NORMALIZE) ? 1 : 0;
  p.out_scale = 1.f;
  p.pair_q = pair_q;
  p.pair_d = pair_d;
  p.nunits = num_pairs;
  p.nc = 1;
  p.LU = pl.LU;
  p.QPG = 1;
  p.ngroups = num_pairs;
  p.ndocs_pg = 1;
  p.R = 1;
  p.NR = 1;
  p.xcd_map = 0;
  p.out = out;
  p.osq = 1;
  p.osd = 0;
  return launch_dense(Q->dtype, pl, p, num_pairs, (hipStream_t)stream);
}

int lik_plaid_maxsim(const lik_seqs_t* Q, const lik_plaid_docs_t* docs, uint32_t flags, float* out,
                     int64_t out_stride_q, int64_t out_stride_d, lik_stream_t stream) {
  int rc;
  if ((rc = check_seqs(Q)) != LIK_OK) return rc;
  if (!docs || docs->n < 0) return LIK_ERR_INVALID;
  if (Q->dtype != LIK_BF16 && Q->dtype != LIK_F16) return LIK_ERR_UNSUPPORTED;
  if (docs->nbits != 2 && docs->nbits != 4 && docs->nbits != 8) return LIK_ERR_INVALID;
  if (docs->dim != Q->dim || Q->dim % 8 != 0) return LIK_ERR_INVALID;
  if (docs->n_buckets < 1 || docs->n_buckets > 256 || !docs->bucket_weights) return LIK_ERR_INVALID;
  if (!docs->cu_seqlens && !docs->lengths) return LIK_ERR_INVALID;
  if (docs->centroid_dtype != LIK_BF16 && docs->centroid_dtype != LIK_F16 && docs->centroid_dtype != LIK_F32)
    return LIK_ERR_UNSUPPORTED;
  if ((flags & LIK_KD_LAYOUT) || Q->mask || Q->token_scale) return LIK_ERR_INVALID;
  if (Q->n == 0 || docs->n == 0) return LIK_OK;
  if (!out || !docs->codes || !docs->residuals || !docs->centroids || docs->n_centroids < 1)
    return LIK_ERR_INVALID;
  const int ceb = elem_bytes(docs->centroid_dtype);
  if (((uintptr_t)docs->centroids) % 16 != 0 || (docs->cent_stride * ceb) % 16 != 0) return LIK_ERR_UNSUPPORTED;
  if (((uintptr_t)docs->residuals) % 8 != 0 || docs->res_stride_tok % docs->nbits != 0)
    return LIK_ERR_UNSUPPORTED;
  if (docs->res_stride_tok * 8 < (int64_t)docs->dim * docs->nbits) return LIK_ERR_INVALID;

  Plan pl;
  if ((rc = make_plan(Q->dtype, Q->dim, Q->n, Q->len, false, pl)) != LIK_OK) return rc;
  if (pl.dpad > 256) return LIK_ERR_UNSUPPORTED;
  if (pl.nc != 1) return LIK_ERR_UNSUPPORTED;  // Lq > 512: chunk on the caller side
  Params p{};
  p.q = to_dev(*Q);
  p.pl.codes = docs->codes;
  p.pl.res = docs->residuals;
  p.pl.cu = docs->cu_seqlens;
  p.pl.lengths = docs->lengths;
  p.pl.n = docs->n;
  p.pl.L = docs->max_len;
  p.pl.codes_sn = docs->codes_stride_n;
  p.pl.res_st = docs->res_stride_tok;
  p.pl.cent = (const char*)docs->centroids;
  p.pl.cent_sb = docs->cent_stride * ceb;
  p.pl.ncent = docs->n_centroids;
  p.pl.bw = docs->bucket_weights;
  p.pl.nb = docs->n_buckets;
  p.pl.nbits = docs->nbits;
  p.normalize = (flags & LIK_NORMALIZE) ? 1 : 0;
  p.out_scale = 1.f;
  p.nunits = pl.nunits;
  p.nc = 1;
  p.LU = pl.LU;
  p.QPG = pl.QPG;
  p.ngroups = pl.ngroups;
  p.kd_K = 0;
  p.ndocs_pg = docs->n;
  p.out = out;
  p.osq = out_stride_q;
  p.osd = out_stride_d;
  p.R = pick_R(p.ngroups, p.ndocs_pg);
  p.NR = (p.ndocs_pg + p.R - 1) / p.R;
  p.xcd_map = p.NR >= 8 ? 1 : 0;
  const int64_t nb = p.xcd_map ? p.ngroups * ((p.NR + 7) / 8) * 8 : p.ngroups * p.NR;
  return launch_plaid(Q->dtype, docs->centroid_dtype, pl, p, nb, (hipStream_t)stream);
}

}  // extern "C"
