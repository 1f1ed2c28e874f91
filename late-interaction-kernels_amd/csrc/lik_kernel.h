// The MaxSim tile kernel (included by lik_maxsim.hip after Params / SeqDev /
// PlaidDev / KT are defined).
//
// Per workgroup: W wavefronts, one per SIMD; wave w owns NSUB blocks of 32
// query-token columns as MFMA B-fragments in VGPRs. The workgroup walks its
// documents as a flat sequence of 32-token tiles. Iteration i of the main
// loop is a software pipeline over four tiles:
//
//   MFMA      tile i     LDS[i%2]            -> accumulator set i%2
//   epilogue  tile i-1   accumulator set (i-1)%2 -> running max (+ doc end)
//   commit    tile i+1   staged VGPRs -> LDS[(i+1)%2] (+ row norm / mask bias)
//   fetch     tile i+3   buffer loads -> staging VGPRs (2-deep ring)
//   [PLAID:   codes of tile i+4; tile i+3's fetch gathers centroids by code]
//   barrier
//
// so the epilogue VALU work of one tile runs under the next tile's MFMAs and
// every global load has two iterations to land. Loads are raw buffer loads:
// rows past a document's end (and dims past d) fall outside the buffer range
// and read as 0 without branches. Per-document metadata is read through
// the workgroup's per-doc table, staged in LDS before the loop.
#pragma once
#include "lik_params.h"

namespace lik {

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t nbytes) {
  // dword3 0x00020000: DATA_FORMAT=32 (untyped raw access), stride 0 -> byte range check
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)nbytes, 0x00020000);
}
constexpr uint32_t kOOB = 0xffffffffu;  // offset guaranteed >= num_records -> loads return 0

__device__ __forceinline__ uint32_t sat_u32(int64_t x) {
  return x < 0 ? 0u : (x >= 0xffffffffLL ? 0xffffffffu : (uint32_t)x);
}
__device__ __forceinline__ uint32_t span_bytes(int64_t len, int64_t stride, int64_t elem) {
  // bytes from element 0 to the end of element len-1 of a strided row
  return len <= 0 ? 0u : sat_u32(((len - 1) * stride + 1) * elem);
}

// A tile of the workgroup's sequence: tile t of the m-th non-empty document.
// Everything else about the document lives in the LDS table s_nz.
struct Tile {
  int m;    // index into s_nz; >= nnz: past the end
  int t;    // tile index within the doc
  int len;  // doc length in tokens
};
struct DocInfo {
  int k;      // doc index within the workgroup's range (jl - jl0)
  int len;    // tokens
  int start;  // packed layouts: first token row
  bool holes; // dense + mask: a dropped token inside [0, len)
};

constexpr int kRMax = 512;  // docs per workgroup (host caps R)

// FEAT: features compiled in (a cleared bit removes the code path; the host
// picks an instantiation whose bits cover the call): F_MASK doc mask,
// F_TS per-token doc scale, F_NORM L2 normalise, F_CU packed docs.
enum { F_MASK = 1, F_TS = 2, F_NORM = 4, F_CU = 8, F_ALL = 15 };

template <int EK, int DPAD, int W, int NSUB, int SRC, int CD, int FEAT>
__global__ void __launch_bounds__(W * 64) maxsim_kernel(const Params p) {
  using T = KT<EK, DPAD>;
  constexpr int NT = W * 64;
  constexpr int COLS = W * NSUB * 32;
  constexpr int KS = T::KSTEPS;
  constexpr int FV = T::FRAG_V;
  constexpr int SCPR = SRC == SRC_DENSE ? T::CPR : DPAD / 8;  // 16-B staging chunks per row
  constexpr int NCH = (32 * SCPR + NT - 1) / NT;
  constexpr bool FULLCH = (32 * SCPR) % NT == 0;
  constexpr int NCV = (SRC == SRC_PLAID && CD == EK_F32) ? 2 : 1;
  constexpr int CSZ = CD == EK_F32 ? 4 : 2;
  constexpr float NEG_INF = -__builtin_huge_valf();
  static_assert(SRC == SRC_DENSE || (!T::SPLIT && EK != EK_FP8), "PLAID computes in bf16/f16");

  __shared__ __attribute__((aligned(16))) char s_tile[2][T::NARR][T::TILE_B];
  __shared__ __attribute__((aligned(16))) float s_rs[3][32];
  __shared__ __attribute__((aligned(16))) float s_rb[3][32];
  // per-unit partial sums of one doc: unit t owns kmax slots, one per 32-column
  // block it touches; QPG * kmax <= 2*COLS + COLS/32 for any unit length.
  __shared__ float s_part[2 * COLS + COLS / 32 + 2];
  __shared__ float s_bw[SRC == SRC_PLAID ? 256 : 1];
  __shared__ int32_t s_dstart[kRMax];
  __shared__ int32_t s_dlen[kRMax];  // length | holes << 31
  __shared__ __attribute__((aligned(16))) i32x4 s_nz[kRMax];  // {k, length | holes << 31, start, 0}
  __shared__ int s_nnz;

  const bool f_mask = (FEAT & F_MASK) && p.d.mask != nullptr;
  const bool f_ts = (FEAT & F_TS) && p.d.ts != nullptr;
  const bool f_norm = (SRC == SRC_PLAID || (FEAT & F_NORM)) && p.normalize;
  const bool f_cu = (FEAT & F_CU) && p.d.cu != nullptr;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wv = tid >> 6, h = lane >> 5, l32 = lane & 31;
  const int kmax = (p.LU + 31) / 32 + 1;

  int64_t g, r;
  {
    const int64_t b = blockIdx.x;
    if (p.xcd_map) {
      // Dispatch is round-robin over the 8 XCDs: every XCD gets whole doc
      // ranges, and all column groups of one range land on the same XCD back
      // to back, so the range's tiles are fetched into that XCD's L2 once.
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
        if (f_norm) ss += chunk_sumsq<EK>(raw[c]);
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
    float sc = f_norm ? inv_norm(ss) : 1.f;
    if (valid && p.q.ts) sc *= p.q.ts[q * p.q.tsn + tok * p.q.tsl];
    qsc[sub] = valid ? sc : 0.f;
  }

  // ---------------- document range and tile cursor ----------------
  const int64_t jl0 = r * (int64_t)p.R;
  const int64_t jl1 = (jl0 + p.R < p.ndocs_pg) ? jl0 + p.R : p.ndocs_pg;
  const int64_t kd_base = p.kd_K ? (g / p.nc) * p.kd_K : 0;  // KD: one query per group
  auto dglob = [&](int64_t jl) -> int64_t {
    if (p.pair_d) {
      const int64_t pd = p.pair_d[g];
      return (pd >= 0 && pd < p.d.n) ? pd : -1;
    }
    return kd_base + jl;
  };
  auto unit_of = [&](int t) -> int64_t { return p.pair_q ? g : g * p.QPG + t; };

  // Per-doc metadata for this workgroup's range, staged once in LDS so the
  // tile cursor never issues a vector load inside the pipelined loop; then
  // wavefront 0 compacts the non-empty docs into s_nz (ballot + popcount).
  const int nloc = (int)(jl1 - jl0);
  for (int k = tid; k < nloc; k += NT) {
    const int64_t jl = jl0 + k;
    const int64_t dg = dglob(jl);
    const int64_t L = doc_len<SRC>(p, dg);
    int32_t start = 0;
    bool holes = false;
    if (dg >= 0) {
      if constexpr (SRC == SRC_DENSE) {
        if (f_cu) start = p.d.cu[dg];
        holes = f_mask && p.holes != nullptr && p.holes[dg] != 0;
      } else {
        if (p.pl.cu) start = p.pl.cu[dg];
      }
    }
    s_dstart[k] = start;
    s_dlen[k] = (int32_t)L | (holes ? (int32_t)0x80000000 : 0);
    if (L == 0) {
      for (int t = 0; t < p.QPG; ++t) {
        const int64_t u = unit_of(t);
        if (u < p.nunits) p.out[u * p.osq + jl * p.osd] = 0.f;
      }
    }
  }
  __syncthreads();
  if (wv == 0) {
    int base = 0;
    for (int k0 = 0; k0 < nloc; k0 += 64) {
      const int k = k0 + lane;
      const int v = k < nloc ? s_dlen[k] : 0;
      const bool nz = (v & 0x7fffffff) > 0;
      const uint64_t bal = __ballot(nz);
      const int pos = base + (int)__popcll(bal & ((1ull << lane) - 1ull));
      if (nz) s_nz[pos] = (i32x4){k, v, s_dstart[k], 0};
      base += (int)__popcll(bal);
    }
    if (lane == 0) s_nnz = base;
  }
  __syncthreads();
  const int nnz = __builtin_amdgcn_readfirstlane(s_nnz);
  if (nnz == 0) return;

  auto doc_info = [&](int m) -> DocInfo {
    const i32x4 e = s_nz[m];
    DocInfo d;
    d.k = __builtin_amdgcn_readfirstlane(e[0]);
    const int v = __builtin_amdgcn_readfirstlane(e[1]);
    d.len = v & 0x7fffffff;
    d.holes = v < 0;
    d.start = __builtin_amdgcn_readfirstlane(e[2]);
    return d;
  };
  auto tile_at = [&](int m) -> Tile {
    Tile x;
    x.m = m;
    x.t = 0;
    x.len = m < nnz ? doc_info(m).len : 0;
    return x;
  };
  auto tile_next = [&](const Tile& c) -> Tile {
    if (c.m >= nnz) return c;
    if ((c.t + 1) * 32 < c.len) {
      Tile n = c;
      n.t = c.t + 1;
      return n;
    }
    return tile_at(c.m + 1);
  };

  // ---------------- staging: fetch (global -> VGPR ring) and commit (-> LDS) ----------------
  u32x4 st[2][NCH][NCV];
  uint32_t sm[SRC == SRC_DENSE ? 2 : 1][NCH];     // dense: mask byte per row
  float sts[SRC == SRC_DENSE ? 2 : 1][NCH];       // dense fp8: token scale per row
  uint32_t sb0[SRC == SRC_PLAID ? 2 : 1][NCH];    // PLAID: residual bits (low)
  uint32_t sb1[SRC == SRC_PLAID ? 2 : 1][NCH];    // PLAID: residual bits (high)
  int32_t scode[SRC == SRC_PLAID ? 2 : 1][NCH];   // PLAID: centroid code per row

  auto chunk_geom = [&](int i, int& row, int& cc, bool& inr) {
    const int c = tid + i * NT;
    row = c / SCPR;
    cc = c % SCPR;
    inr = FULLCH || c < 32 * SCPR;
  };

  // PLAID phase A: centroid codes of tile x
  auto fetch_codes = [&](auto SS, const Tile& x) {
    if constexpr (SRC == SRC_PLAID) {
      constexpr int S = decltype(SS)::value;
      if (x.m >= nnz) return;
      const DocInfo di = doc_info(x.m);
      const int64_t tok0 = p.pl.cu ? (int64_t)di.start : dglob(jl0 + di.k) * p.pl.codes_sn;
      const __amdgpu_buffer_rsrc_t rc = make_rsrc(p.pl.codes + tok0, sat_u32((int64_t)x.len * 4));
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        int row, cc;
        bool inr;
        chunk_geom(i, row, cc, inr);
        const uint32_t off = inr ? (uint32_t)(x.t * 32 + row) * 4u : kOOB;
        scode[S][i] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rc, off, 0, 0);
      }
    }
  };

  // phase B (dense: the only phase): token data of tile x into slot S
  auto fetch_data = [&](auto SS, const Tile& x) {
    constexpr int S = decltype(SS)::value;
    if (x.m >= nnz) return;
    const DocInfo di = doc_info(x.m);
    const int64_t doc = dglob(jl0 + di.k);
    if constexpr (SRC == SRC_DENSE) {
      const char* base = f_cu ? p.d.data + (int64_t)di.start * p.d.sl_b : p.d.data + doc * p.d.sn_b;
      const __amdgpu_buffer_rsrc_t rd =
          make_rsrc(base, sat_u32((int64_t)(x.len - 1) * p.d.sl_b + (int64_t)p.d.dim * T::IN_B));
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        int row, cc;
        bool inr;
        chunk_geom(i, row, cc, inr);
        const int64_t tok = (int64_t)x.t * 32 + row;
        const bool ok = inr && tok < x.len && cc * T::CHUNK_E < p.d.dim;
        const uint32_t off = ok ? sat_u32(tok * p.d.sl_b + cc * 16) : kOOB;
        st[S][i][0] = __builtin_amdgcn_raw_buffer_load_b128(rd, off, 0, 0);
      }
      if (f_mask) {
        const __amdgpu_buffer_rsrc_t rm =
            make_rsrc(p.d.mask + doc * p.d.msn, span_bytes(x.len, p.d.msl, 1));
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
          int row, cc;
          bool inr;
          chunk_geom(i, row, cc, inr);
          const int64_t tok = (int64_t)x.t * 32 + row;
          const uint32_t off = (inr && tok < x.len) ? sat_u32(tok * p.d.msl) : kOOB;
          sm[S][i] = __builtin_amdgcn_raw_buffer_load_b8(rm, off, 0, 0);
        }
      }
      if (f_ts) {
        const __amdgpu_buffer_rsrc_t rt =
            make_rsrc(p.d.ts + doc * p.d.tsn, span_bytes(x.len, p.d.tsl, 4));
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
          int row, cc;
          bool inr;
          chunk_geom(i, row, cc, inr);
          const int64_t tok = (int64_t)x.t * 32 + row;
          const uint32_t off = (inr && tok < x.len) ? sat_u32(tok * p.d.tsl * 4) : kOOB;
          sts[S][i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rt, off, 0, 0));
        }
      }
    } else {
      const int64_t tok0 = p.pl.cu ? (int64_t)di.start : doc * p.pl.codes_sn;
      const __amdgpu_buffer_rsrc_t rcent = make_rsrc(p.pl.cent, sat_u32(p.pl.ncent * p.pl.cent_sb));
      const __amdgpu_buffer_rsrc_t rres =
          make_rsrc(p.pl.res + tok0 * p.pl.res_st, sat_u32((int64_t)x.len * p.pl.res_st));
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        int row, cc;
        bool inr;
        chunk_geom(i, row, cc, inr);
        const int64_t tl = (int64_t)x.t * 32 + row;
        const bool ok = inr && tl < x.len && cc * 8 < p.q.dim;
        int64_t code = scode[S][i];
        code = (code < 0 || code >= p.pl.ncent) ? 0 : code;
        const uint32_t coff = ok ? sat_u32(code * p.pl.cent_sb + (int64_t)cc * 8 * CSZ) : kOOB;
        st[S][i][0] = __builtin_amdgcn_raw_buffer_load_b128(rcent, coff, 0, 0);
        if constexpr (NCV > 1) st[S][i][1] = __builtin_amdgcn_raw_buffer_load_b128(rcent, coff + 16u, 0, 0);
        const uint32_t roff = ok ? sat_u32(tl * p.pl.res_st + (int64_t)cc * p.pl.nbits) : kOOB;
        if (p.pl.nbits == 2) {
          sb0[S][i] = __builtin_amdgcn_raw_buffer_load_b16(rres, roff, 0, 0);
          sb1[S][i] = 0;
        } else if (p.pl.nbits == 4) {
          sb0[S][i] = __builtin_amdgcn_raw_buffer_load_b32(rres, roff, 0, 0);
          sb1[S][i] = 0;
        } else {
          const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rres, roff, 0, 0);
          sb0[S][i] = v[0];
          sb1[S][i] = v[1];
        }
      }
    }
  };

  auto commit = [&](auto SS, const Tile& x, int buf, int rslot) {
    constexpr int S = decltype(SS)::value;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      int row, cc;
      bool inr;
      chunk_geom(i, row, cc, inr);
      const bool live = x.t * 32 + row < x.len;
      if constexpr (SRC == SRC_DENSE) {
        float ss = 0.f;
        if (f_norm) {
          ss = chunk_sumsq<EK>(st[S][i][0]);
#pragma unroll
          for (int o = 1; o < SCPR; o <<= 1) ss += __shfl_xor(ss, o);
        }
        if (inr) {
          char* rowp = s_tile[buf][0] + row * T::ROW_B;
          if constexpr (T::SPLIT) {
            u32x2 hi, lo;
            split4(st[S][i][0], hi, lo);
            *(u32x2*)(rowp + cc * 8) = hi;
            *(u32x2*)(s_tile[buf][1] + row * T::ROW_B + cc * 8) = lo;
          } else {
            *(u32x4*)(rowp + cc * 16) = st[S][i][0];
          }
          if (cc == 0) {
            const bool ok = live && (!f_mask || (sm[S][i] & 0xffu) != 0);
            s_rs[rslot][row] = (f_norm ? inv_norm(ss) : 1.f) * (f_ts ? sts[S][i] : 1.f);
            s_rb[rslot][row] = ok ? 0.f : NEG_INF;
          }
        }
      } else {
        const uint32_t bmask = (1u << p.pl.nbits) - 1u;
        const uint64_t bits = ((uint64_t)sb1[S][i] << 32) | sb0[S][i];
        float x8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float cv;
          if constexpr (CD == EK_F32) cv = __uint_as_float(st[S][i][e >> 2][e & 3]);
          else if constexpr (CD == EK_BF16)
            cv = (e & 1) ? bf16hi_to_f32(st[S][i][0][e >> 1]) : bf16lo_to_f32(st[S][i][0][e >> 1]);
          else
            cv = f16_to_f32((uint16_t)((e & 1) ? (st[S][i][0][e >> 1] >> 16) : (st[S][i][0][e >> 1] & 0xffffu)));
          uint32_t bc = (uint32_t)(bits >> (e * p.pl.nbits)) & bmask;
          bc = bc < (uint32_t)p.pl.nb ? bc : (uint32_t)(p.pl.nb - 1);
          x8[e] = (live && (cc * 8 + e) < p.q.dim) ? cv + s_bw[bc] : 0.f;
        }
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(x8[e], x8[e], ss);
#pragma unroll
        for (int o = 1; o < SCPR; o <<= 1) ss += __shfl_xor(ss, o);
        const float sc = p.normalize ? inv_norm(ss) : 1.f;
        if (inr) {
          u32x4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if constexpr (EK == EK_F16)
              w[e] = f32_to_f16_bits(x8[2 * e] * sc) | (f32_to_f16_bits(x8[2 * e + 1] * sc) << 16);
            else
              w[e] = f32_to_bf16_bits(x8[2 * e] * sc) | (f32_to_bf16_bits(x8[2 * e + 1] * sc) << 16);
          }
          *(u32x4*)(s_tile[buf][0] + row * T::ROW_B + cc * 16) = w;
          if (cc == 0) {
            s_rs[rslot][row] = 1.f;
            s_rb[rslot][row] = live ? 0.f : NEG_INF;
          }
        }
      }
    }
  };

  // ---------------- compute pieces ----------------
  f32x16 acc[2][NSUB];
  float m[NSUB];
#pragma unroll
  for (int sub = 0; sub < NSUB; ++sub) m[sub] = NEG_INF;
  const bool dense_fix = SRC == SRC_DENSE && (f_norm || f_ts);

  auto mma_tile = [&](auto PP, int buf) {
    constexpr int P = decltype(PP)::value;
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
          if (ks == 0) {
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[P][sub][e] = 0.f;
          }
          mfma32<EK>(acc[P][sub], a, bq[sub][ks]);
          mfma32<EK>(acc[P][sub], a, &bql[sub][ks]);
          mfma32<EK>(acc[P][sub], &al, bq[sub][ks]);
        }
      } else {
#pragma unroll
        for (int sub = 0; sub < NSUB; ++sub) {
          if (ks == 0) {
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[P][sub][e] = 0.f;
          }
          mfma32<EK>(acc[P][sub], a, bq[sub][ks]);
        }
      }
    }
  };

  auto epilogue = [&](auto PP, const Tile& x, int rslot) {
    constexpr int P = decltype(PP)::value;
    const bool partial = (x.t + 1) * 32 > x.len;
    bool fix = dense_fix || partial;
    const DocInfo di = doc_info(x.m);
    if constexpr (SRC == SRC_DENSE) fix = fix || di.holes;
    if (fix) {
      f32x4 sc[4], bi[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sc[j] = *(const f32x4*)&s_rs[rslot][8 * j + 4 * h];
        bi[j] = *(const f32x4*)&s_rb[rslot][8 * j + 4 * h];
      }
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) m[sub] = fmaxf(m[sub], fmaf(acc[P][sub][4 * j + e], sc[j][e], bi[j][e]));
    } else {
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
        for (int e = 0; e < 16; ++e) m[sub] = fmaxf(m[sub], acc[P][sub][e]);
    }
    if ((x.t + 1) * 32 >= x.len) {  // last tile of the doc: per-column max -> per-unit sum
      // Columns of one unit are contiguous. A segmented inclusive scan over
      // the 32 columns of each block leaves one partial per (unit, block) at
      // the segment's last lane; partials go to LDS and one thread per unit
      // adds its (at most kmax) partials in block order: deterministic.
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub) {
        const float mm = fmaxf(m[sub], __shfl_xor(m[sub], 32));
        m[sub] = NEG_INF;
        const int blk = wv * NSUB + sub;
        const int col = blk * 32 + l32;
        const int ul = col / p.LU;
        float v = (__builtin_isfinite(mm) && ul < p.QPG) ? mm * qsc[sub] : 0.f;
        const int seg0 = max(ul * p.LU - blk * 32, 0);  // first lane of this lane's unit in the block
#pragma unroll
        for (int d = 1; d < 32; d <<= 1) {
          const float o = __shfl_up(v, d, 32);
          if (l32 - d >= seg0) v += o;
        }
        const bool seg_end = l32 == 31 || col + 1 == (ul + 1) * p.LU;
        if (h == 0 && seg_end && ul < p.QPG) s_part[ul * kmax + (blk - (ul * p.LU) / 32)] = v;
      }
      __syncthreads();
      for (int t = tid; t < p.QPG; t += NT) {
        const int64_t u = unit_of(t);
        if (u < p.nunits) {
          const int nparts = (t * p.LU + p.LU - 1) / 32 - (t * p.LU) / 32 + 1;
          float sum = 0.f;
          for (int k = 0; k < nparts; ++k) sum += s_part[t * kmax + k];
          p.out[u * p.osq + (jl0 + di.k) * p.osd] = sum * p.out_scale;
        }
      }
    }
  };

  // ---------------- prologue ----------------
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  Tile tm1;
  tm1.m = nnz;
  tm1.t = 0;
  tm1.len = 0;
  Tile t0 = tile_at(0);
  Tile t1 = tile_next(t0);
  Tile t2 = tile_next(t1);
  Tile t3 = tile_next(t2);
  Tile t4 = tile_next(t3);
  fetch_codes(I0{}, t0);
  fetch_codes(I1{}, t1);
  fetch_data(I0{}, t0);
  fetch_data(I1{}, t1);
  fetch_codes(I0{}, t2);
  fetch_codes(I1{}, t3);
  int rs_commit = 0;  // s_rs/s_rb slot of the tile committed next
  commit(I0{}, t0, 0, rs_commit);
  rs_commit = 1;
  fetch_data(I0{}, t2);
  __syncthreads();
  int rs_epi = 0;  // slot of the tile whose epilogue runs next

  // ---------------- main loop (unrolled by 2 so register slots are static) ----------------
  auto step = [&](auto PP) -> bool {
    constexpr int P = decltype(PP)::value;
    using IP = std::integral_constant<int, P>;
    using IQ = std::integral_constant<int, 1 - P>;
    if (t0.m < nnz) mma_tile(IP{}, P);
    if (tm1.m < nnz) {
      epilogue(IQ{}, tm1, rs_epi);
      rs_epi = rs_epi == 2 ? 0 : rs_epi + 1;
    }
    if (t0.m >= nnz) return false;
    if (t1.m < nnz) {
      commit(IQ{}, t1, 1 - P, rs_commit);
      rs_commit = rs_commit == 2 ? 0 : rs_commit + 1;
    }
    fetch_data(IQ{}, t3);   // uses codes slot (i+3)%2 == 1-P
    fetch_codes(IP{}, t4);  // codes of tile i+4 into slot P
    __syncthreads();
    tm1 = t0;
    t0 = t1;
    t1 = t2;
    t2 = t3;
    t3 = t4;
    t4 = tile_next(t4);
    return true;
  };
  while (true) {
    if (!step(I0{})) break;
    if (!step(I1{})) break;
  }
}



template <int EK, int DPAD, int W, int NSUB, int SRC, int CD, int FEAT>
int launch_one(const Params& p, int64_t nblocks, hipStream_t s) {
  if constexpr (!cfg_ok<EK, DPAD, NSUB>()) {
    return LIK_ERR_UNSUPPORTED;
  } else {
    if (nblocks <= 0) return LIK_OK;
    if (nblocks > 0x7fffffffLL) return LIK_ERR_UNSUPPORTED;
    hipLaunchKernelGGL((maxsim_kernel<EK, DPAD, W, NSUB, SRC, CD, FEAT>), dim3((unsigned)nblocks), dim3(W * 64), 0, s, p);
    return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
  }
}

// Column-block configurations (W wavefronts x NSUB 32-column blocks each).
template <int EK, int DPAD, int SRC, int CD, int FEAT>
int launch_cfg(const Plan& pl, const Params& p, int64_t nb, hipStream_t s) {
  if (pl.W == 1 && pl.NSUB == 1) return launch_one<EK, DPAD, 1, 1, SRC, CD, FEAT>(p, nb, s);
  if (pl.W == 1 && pl.NSUB == 2) return launch_one<EK, DPAD, 1, 2, SRC, CD, FEAT>(p, nb, s);
  if (pl.W == 1 && pl.NSUB == 4) return launch_one<EK, DPAD, 1, 4, SRC, CD, FEAT>(p, nb, s);
  if (pl.W == 4 && pl.NSUB == 1) return launch_one<EK, DPAD, 4, 1, SRC, CD, FEAT>(p, nb, s);
  if (pl.W == 4 && pl.NSUB == 2) return launch_one<EK, DPAD, 4, 2, SRC, CD, FEAT>(p, nb, s);
  if (pl.W == 4 && pl.NSUB == 4) return launch_one<EK, DPAD, 4, 4, SRC, CD, FEAT>(p, nb, s);
  if (pl.W == 8 && pl.NSUB == 1) return launch_one<EK, DPAD, 8, 1, SRC, CD, FEAT>(p, nb, s);
  if (pl.W == 8 && pl.NSUB == 2) return launch_one<EK, DPAD, 8, 2, SRC, CD, FEAT>(p, nb, s);
  return LIK_ERR_UNSUPPORTED;
}

template <int EK, int SRC, int CD, int FEAT>
int launch_dpad(const Plan& pl, const Params& p, int64_t nb, hipStream_t s) {
  switch (pl.dpad) {
    case 64: return launch_cfg<EK, 64, SRC, CD, FEAT>(pl, p, nb, s);
    case 128: return launch_cfg<EK, 128, SRC, CD, FEAT>(pl, p, nb, s);
    case 256: return launch_cfg<EK, 256, SRC, CD, FEAT>(pl, p, nb, s);
    case 512:
      if constexpr ((EK == EK_BF16 || EK == EK_F16) && SRC == SRC_DENSE)
        return launch_cfg<EK, 512, SRC, CD, FEAT>(pl, p, nb, s);
      else
        return LIK_ERR_UNSUPPORTED;
    default: return LIK_ERR_UNSUPPORTED;
  }
}

// Features a call needs (FEAT bits).
inline int needed_feat(const Params& p) {
  return (p.d.mask ? F_MASK : 0) | (p.d.ts ? F_TS : 0) | (p.normalize ? F_NORM : 0) | (p.d.cu ? F_CU : 0);
}

}  // namespace lik
