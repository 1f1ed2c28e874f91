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
  int m;        // index into s_nz; >= nnz: past the end
  int t;        // tile index within the doc
  int len;      // doc length in tokens
  int k;        // doc index within the workgroup's range (jl - jl0)
  bool holes;   // dense + mask: a dropped token inside [0, len)
  int64_t off;  // dense: byte offset of the doc's token 0 from the data base; PLAID: its first token index
};

constexpr int kRMax = 512;  // docs per workgroup (host caps R)

#ifdef LIK_PROF
// Profiling builds only: per-phase cycle totals of the tile loop, summed over
// all waves (lane 0 of each wave adds its totals at exit).
#define LIK_PROF_DECL unsigned long long prof_acc[6] = {0, 0, 0, 0, 0, 0}; unsigned long long prof_t = __builtin_readcyclecounter();
#define LIK_PROF_MARK(k) do { const unsigned long long t_ = __builtin_readcyclecounter(); prof_acc[k] += t_ - prof_t; prof_t = t_; } while (0)
#define LIK_PROF_FLUSH() do { if (lane == 0 && p.prof) { for (int k_ = 0; k_ < 6; ++k_) atomicAdd(&p.prof[k_], prof_acc[k_]); atomicAdd(&p.prof[6], 1ull); } } while (0)
#else
#define LIK_PROF_DECL
#define LIK_PROF_MARK(k) do { } while (0)
#define LIK_PROF_FLUSH() do { } while (0)
#endif

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
  __shared__ __attribute__((aligned(16))) float s_rs[3][32];  // per-row scale (normalise / fp8 token scale)
  __shared__ uint32_t s_tb[3];  // per-tile row-validity words of docs with mask holes
  // Finished documents: per-column maxima (already scaled, 0 for invalid
  // columns) of the last 16 docs and their local indices. A half (8 docs) is
  // summed per unit and written out one iteration after it fills.
  constexpr int NSLOT = 16;
  __shared__ __attribute__((aligned(16))) float s_colb[NSLOT][COLS];
  __shared__ int s_slotk[NSLOT];
  __shared__ float s_bw[SRC == SRC_PLAID ? 256 : 1];
  __shared__ int64_t s_doff[kRMax];  // dense: byte offset of token 0; PLAID: first token index
  __shared__ float* s_outp[COLS];      // per unit of the group: &out[u, jl0] (null: no unit)
  __shared__ int32_t s_dlen[kRMax];  // length | holes << 31
  __shared__ __attribute__((aligned(16))) i32x4 s_nz[kRMax];  // {k, length | holes << 31, start, 0}
  __shared__ int s_nnz, s_ntiles;

  const bool f_mask = (FEAT & F_MASK) && p.d.mask != nullptr;
  const bool f_ts = (FEAT & F_TS) && p.d.ts != nullptr;
  const bool f_norm = (SRC == SRC_PLAID || (FEAT & F_NORM)) && p.normalize;
  const bool f_cu = (FEAT & F_CU) && p.d.cu != nullptr;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wv = tid >> 6, h = lane >> 5, l32 = lane & 31;

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

  // ---------------- document range and tile cursor ----------------
  const int64_t jl0 = r * (int64_t)p.R;
  const int64_t jl1 = (jl0 + p.R < p.ndocs_pg) ? jl0 + p.R : p.ndocs_pg;
  const int64_t kd_base = p.kd_K ? (g / p.nc) * p.kd_K : 0;  // KD: one query per group
  int64_t pair_doc = -1;
  if (p.pair_d) {
    const int64_t pd = p.pair_d[g];
    pair_doc = (pd >= 0 && pd < p.d.n) ? pd : -1;
  }
  auto dglob = [&](int64_t jl) -> int64_t { return p.pair_d ? pair_doc : kd_base + jl; };
  auto unit_of = [&](int t) -> int64_t { return p.pair_q ? g : g * p.QPG + t; };

  // Output row pointers of the group's units (shifted to doc jl0), so the doc
  // flush needs only the column stride.
  for (int t = tid; t < COLS; t += NT) {
    const int64_t u = unit_of(t);
    s_outp[t] = (t < p.QPG && u < p.nunits) ? p.out + u * p.osq + jl0 * p.osd : nullptr;
  }
  __syncthreads();
  // Per-doc metadata for this workgroup's range, staged once in LDS so the
  // tile cursor never issues a vector load inside the pipelined loop; then
  // wavefront 0 compacts the non-empty docs into s_nz (ballot + popcount).
  const int nloc = (int)(jl1 - jl0);
  for (int k = tid; k < nloc; k += NT) {
    const int64_t jl = jl0 + k;
    const int64_t dg = dglob(jl);
    const int64_t L = doc_len<SRC>(p, dg);
    int64_t off = 0;
    bool holes = false, skip = false;
    if (dg >= 0) {
      if constexpr (SRC == SRC_DENSE) {
        off = f_cu ? (int64_t)p.d.cu[dg] * p.d.sl_b : dg * p.d.sn_b;
        const bool h = p.holes != nullptr && p.holes[dg] != 0;
        holes = f_mask && h;
        // two-launch mask handling: 1 = docs without holes only, 2 = docs with holes only
        skip = (p.doc_filter == 1 && h) || (p.doc_filter == 2 && !h);
      } else {
        off = p.pl.cu ? (int64_t)p.pl.cu[dg] : dg * p.pl.codes_sn;
      }
    }
    s_doff[k] = off;
    s_dlen[k] = skip ? 0 : ((int32_t)L | (holes ? (int32_t)0x80000000 : 0));
    if (L == 0 && !skip) {
      for (int t = 0; t < p.QPG; ++t)
        if (float* o = s_outp[t]) o[k * p.osd] = 0.f;
    }
  }
  __syncthreads();
  if (wv == 0) {
    int base = 0, ntl = 0;
    for (int k0 = 0; k0 < nloc; k0 += 64) {
      const int k = k0 + lane;
      const int v = k < nloc ? s_dlen[k] : 0;
      const int L = v & 0x7fffffff;
      const bool nz = L > 0;
      const uint64_t bal = __ballot(nz);
      const int pos = base + (int)__popcll(bal & ((1ull << lane) - 1ull));
      if (nz) s_nz[pos] = (i32x4){k, v, (int)(uint32_t)s_doff[k], (int)(s_doff[k] >> 32)};
      base += (int)__popcll(bal);
      int nt = (L + 31) >> 5;
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) nt += __shfl_xor(nt, o);
      ntl += nt;
    }
    if (lane == 0) {
      s_nnz = base;
      s_ntiles = ntl;
    }
  }
  __syncthreads();
  const int nnz = __builtin_amdgcn_readfirstlane(s_nnz);
  const int ntiles = __builtin_amdgcn_readfirstlane(s_ntiles);
  if (nnz == 0) return;

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


  // Cursor over the workgroup's tile sequence: tile t of the m-th non-empty
  // doc. The doc fields are refreshed from the LDS table only when the cursor
  // crosses a document boundary.
  auto cur_load = [&](Tile& c, int m) {
    c.m = m;
    c.t = 0;
    if (m < nnz) {
      const i32x4 e = s_nz[m];
      c.k = __builtin_amdgcn_readfirstlane(e[0]);
      const int v = __builtin_amdgcn_readfirstlane(e[1]);
      c.len = v & 0x7fffffff;
      c.holes = v < 0;
      c.off = (int64_t)(uint32_t)__builtin_amdgcn_readfirstlane(e[2]) |
              ((int64_t)__builtin_amdgcn_readfirstlane(e[3]) << 32);
    } else {
      c.k = 0;
      c.len = 0;
      c.holes = false;
      c.off = 0;
    }
  };
  auto cur_adv = [&](Tile& c) {
    if (c.m >= nnz) return;
    if ((c.t + 1) * 32 < c.len) ++c.t;
    else cur_load(c, c.m + 1);
  };

  // ---------------- staging: fetch (global -> VGPR ring) and commit (-> LDS) ----------------
  u32x4 st[2][NCH][NCV];
  uint32_t sm[SRC == SRC_DENSE ? 2 : 1];          // dense + mask holes: the tile's row-validity word
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
      const int64_t tok0 = x.off;
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
    if constexpr (SRC == SRC_DENSE) {
      const int64_t doc = dglob(jl0 + x.k);
      const char* base = p.d.data + x.off;
      const __amdgpu_buffer_rsrc_t rd =
          make_rsrc(base, sat_u32((int64_t)(x.len - 1) * p.d.sl_b + (int64_t)p.d.dim * T::IN_B));
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        int row, cc;
        bool inr;
        chunk_geom(i, row, cc, inr);
        const int64_t tok = (int64_t)x.t * 32 + row;
        const bool ok = inr && tok < x.len && cc * T::CHUNK_E < p.d.dim;
        // valid offsets are < the 4 GiB buffer range, so 32-bit arithmetic is exact
        const uint32_t off = ok ? (uint32_t)tok * (uint32_t)p.d.sl_b + (uint32_t)(cc * 16) : kOOB;
        st[S][i][0] = __builtin_amdgcn_raw_buffer_load_b128(rd, off, 0, 0);
      }
      if (f_mask && x.holes) {  // prefix-valid docs need no validity word
        const __amdgpu_buffer_rsrc_t rm = make_rsrc(p.tbits + doc * p.tbits_sn, sat_u32(p.tbits_sn * 4));
        sm[S] = __builtin_amdgcn_raw_buffer_load_b32(rm, (uint32_t)x.t * 4u, 0, 0);
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
      const int64_t tok0 = x.off;
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
    if constexpr (SRC == SRC_DENSE) {
      if (f_mask && x.holes && tid == 0) s_tb[rslot] = sm[S];
    }
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
          if (cc == 0 && (f_norm || f_ts)) s_rs[rslot][row] = (f_norm ? inv_norm(ss) : 1.f) * (f_ts ? sts[S][i] : 1.f);
        }
      } else {
        (void)rslot;
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
        }
      }
    }
  };

  // ---------------- compute pieces ----------------
  // W=8: two waves of one workgroup share a SIMD, so each wave double-buffers
  // its accumulators and overlaps tile i's MFMAs with tile i-1's epilogue.
  // W<=4: a single accumulator set keeps a wave under 256 registers, so two
  // workgroups fit per CU and hide each other's epilogues and barriers.
#ifndef LIK_DACC_W8
#define LIK_DACC_W8 1
#endif
  constexpr bool DACC = W == 8 && LIK_DACC_W8;
  f32x16 acc[DACC ? 2 : 1][NSUB];
  float m[NSUB];
#pragma unroll
  for (int sub = 0; sub < NSUB; ++sub) m[sub] = NEG_INF;
  const bool dense_fix = SRC == SRC_DENSE && (f_norm || f_ts);

  auto mma_tile = [&](auto PP, int buf) {
    constexpr int P = DACC ? decltype(PP)::value : 0;
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

  int nend = 0;  // documents finished so far

  // Sum the per-column maxima of finished docs [s0, s0+n) per unit and write
  // scores: one thread per (doc, unit), columns added in a fixed (rotated)
  // order, so results are bitwise reproducible.
  auto flush = [&](int s0, int n) {
    const int tasks = n * p.QPG;
    for (int task = tid; task < tasks; task += NT) {
      const int sl = (s0 + task / p.QPG) % NSLOT;
      const int t = task % p.QPG;
      float* const orow = s_outp[t];
      if (!orow) continue;
      const float* cv = &s_colb[sl][t * p.LU];
      float sum = 0.f;
      if ((p.LU & 3) == 0) {
        const int nv = p.LU >> 2;
        int c = t % nv;
        for (int j = 0; j < nv; ++j) {
          const f32x4 v = *(const f32x4*)(cv + 4 * c);
          sum += v[0];
          sum += v[1];
          sum += v[2];
          sum += v[3];
          c = (c + 1 == nv) ? 0 : c + 1;
        }
      } else {
        for (int j = 0; j < p.LU; ++j) sum += cv[j];
      }
      orow[s_slotk[sl] * p.osd] = sum * p.out_scale;
    }
  };

  auto epilogue = [&](auto PP, const Tile& x, int rslot) {
    constexpr int P = DACC ? decltype(PP)::value : 0;
    // Row validity: rows past the doc end, and (dense + mask holes) rows whose
    // bit in the tile's validity word is clear, never win the max.
    const int nv = x.len - x.t * 32;
    bool holes = false;
    if constexpr (SRC == SRC_DENSE) holes = f_mask && x.holes;
    const uint32_t vbits = (holes ? s_tb[rslot] : 0xffffffffu) & (nv >= 32 ? 0xffffffffu : ((1u << nv) - 1u));
    if (dense_fix) {
      f32x4 sc[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) sc[j] = *(const f32x4*)&s_rs[rslot][8 * j + 4 * h];
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float v = acc[P][sub][4 * j + e] * sc[j][e];
            m[sub] = fmaxf(m[sub], ((vbits >> (8 * j + 4 * h + e)) & 1u) ? v : NEG_INF);
          }
    } else if (vbits != 0xffffffffu) {
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            m[sub] = fmaxf(m[sub], ((vbits >> (8 * j + 4 * h + e)) & 1u) ? acc[P][sub][4 * j + e] : NEG_INF);
    } else {
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
        for (int e = 0; e < 16; ++e) m[sub] = fmaxf(m[sub], acc[P][sub][e]);
    }
    if ((x.t + 1) * 32 >= x.len) {  // last tile of the doc: park the per-column maxima
      const int sl = nend % NSLOT;
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub) {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(m[sub]), __float_as_uint(m[sub]), false, false);
        const float mm = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));  // max over lanes l, l^32
        if (h == 0) s_colb[sl][(wv * NSUB + sub) * 32 + l32] = __builtin_isfinite(mm) ? mm * qsc[sub] : 0.f;
        m[sub] = NEG_INF;
      }
      if (tid == 0) s_slotk[sl] = x.k;
      ++nend;
    }
  };

  // ---------------- prologue ----------------
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  // cursors: ce epilogue (tile i-1), cm commit (i+1), cf fetch (i+3), cp codes (i+4)
  Tile ce, cm, cf, cp;
  cur_load(ce, 0);
  cm = ce;
  fetch_codes(I0{}, cm);  // tile 0
  fetch_data(I0{}, cm);
  cur_adv(cm);            // tile 1
  fetch_codes(I1{}, cm);
  fetch_data(I1{}, cm);
  cf = cm;
  cur_adv(cf);            // tile 2
  fetch_codes(I0{}, cf);
  cp = cf;
  cur_adv(cp);            // tile 3
  fetch_codes(I1{}, cp);
  commit(I0{}, ce, 0, 0); // tile 0 -> LDS[0], row slot 0
  fetch_data(I0{}, cf);   // tile 2 into slot 0
  cf = cp;                // tile 3
  cur_adv(cp);            // tile 4
  __syncthreads();
  int rs_commit = 1;      // row-scale slot of tile i+1
  int rs_epi = 0;         // row-scale slot of tile i-1
  int flush_half = -1;    // slot half whose flush is due (after the barrier it waited for)

  // ---------------- main loop (unrolled by 2 so register slots are static) ----------------
  LIK_PROF_DECL
  auto step = [&](auto PP, int i) -> bool {
    constexpr int P = decltype(PP)::value;
    using IP = std::integral_constant<int, P>;
    using IQ = std::integral_constant<int, 1 - P>;
    if (flush_half >= 0) {
      flush(flush_half * 8, 8);
      flush_half = -1;
    }
    LIK_PROF_MARK(0);
    const int nend0 = nend;
    if constexpr (DACC) {
      if (i < ntiles) mma_tile(IP{}, P);
      if (i >= 1) {
        epilogue(IQ{}, ce, rs_epi);
        rs_epi = rs_epi == 2 ? 0 : rs_epi + 1;
        cur_adv(ce);
      }
    } else {
      if (i >= 1) {
        epilogue(IQ{}, ce, rs_epi);
        rs_epi = rs_epi == 2 ? 0 : rs_epi + 1;
        cur_adv(ce);
      }
      if (i < ntiles) mma_tile(IP{}, P);
    }
    if (nend != nend0 && (nend & 7) == 0) flush_half = ((nend >> 3) - 1) & 1;
    LIK_PROF_MARK(1);
    if (i >= ntiles) return false;
    if (i + 1 < ntiles) {
      commit(IQ{}, cm, 1 - P, rs_commit);
      rs_commit = rs_commit == 2 ? 0 : rs_commit + 1;
      cur_adv(cm);
    }
    LIK_PROF_MARK(2);
    fetch_data(IQ{}, cf);   // tile i+3 into slot (i+3)%2, codes from slot (i+3)%2
    cur_adv(cf);
    if constexpr (SRC == SRC_PLAID) {
      fetch_codes(IP{}, cp);  // codes of tile i+4 into slot P
      cur_adv(cp);
    }
    LIK_PROF_MARK(3);
    __syncthreads();
    LIK_PROF_MARK(4);
    return true;
  };
  for (int i = 0;; i += 2) {
    if (!step(I0{}, i)) break;
    if (!step(I1{}, i + 1)) break;
  }
  // remaining finished docs: the due half (if any) and the partial half
  __syncthreads();
  if (flush_half >= 0) flush(flush_half * 8, 8);
  if (nend & 7) flush(nend & ~7, nend & 7);
  LIK_PROF_MARK(5);
  LIK_PROF_FLUSH();
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
