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


constexpr int kRMax = 512;  // docs per workgroup (host caps R)


// FEAT: features compiled in (a cleared bit removes the code path; the host
// picks an instantiation whose bits cover the call): F_MASK doc mask,
// F_TS per-token doc scale, F_NORM L2 normalise, F_CU packed docs.
// F_ARGMAX (training forward): also write each (query token, doc) winner's doc-token index.
// F_NORM: normalise query and / or doc tokens (runtime bits); F_NORMQ:
// normalise query tokens only (prologue code, nothing in the tile loop).
enum { F_MASK = 1, F_TS = 2, F_NORM = 4, F_CU = 8, F_ALL = 15, F_ARGMAX = 16, F_NORMQ = 32 };

// Four-wave workgroups of 4 column blocks per wave (dense bf16 / fp16
// scoring without masks, normalisation or argmax, which would not fit) are
// held to 256 registers so that two workgroups share each CU: their
// barriers are independent, so one workgroup's per-tile bookkeeping and
// barrier wait are covered by the other's MFMAs.
template <int EK, int W, int NSUB, int SRC, int FEAT>
constexpr bool two_wg_per_cu() {
  // fp8 also runs 4 x 6: its query fragments take half the registers of
  // 16-bit ones, and a tile holds only two k-steps of MFMA work, so more
  // column blocks per wave amortise the per-tile work (+30% measured)
  return W == 4 && (NSUB == 4 || (NSUB == 6 && EK == EK_FP8)) && SRC == SRC_DENSE &&
         (EK == EK_BF16 || EK == EK_F16 || EK == EK_FP8) && (FEAT & (F_ARGMAX | F_NORM | F_TS | F_MASK)) == 0;
}
// Workgroups per CU of those kernels (fp8 would nearly fit three, but spills
// at 168 VGPRs and measures slower).
template <int EK, int W, int NSUB, int SRC, int FEAT>
constexpr int wg_per_cu() {
  return two_wg_per_cu<EK, W, NSUB, SRC, FEAT>() ? 2 : 1;
}

template <int EK, int DPAD, int W, int NSUB, int SRC, int CD, int FEAT>
__global__ void __launch_bounds__(W * 64)
    __attribute__((amdgpu_waves_per_eu(wg_per_cu<EK, W, NSUB, SRC, FEAT>())))
    maxsim_kernel(const Params p) {
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

  // Direct global -> LDS tile loads (buffer_load ... lds) in the two-workgroup
  // kernel with 256-byte rows: no staging registers, no LDS writes of staged
  // data. A DMA instruction writes 64 x 16 bytes contiguously, so those tiles
  // are unpadded and chunk-major (16-byte chunk c of row r at c * 512 + r * 16),
  // which keeps the A-fragment reads conflict-free; they cycle through 4
  // buffers (tile i multiplied, tiles i+1 .. i+3 landing).
  constexpr bool kDMA = two_wg_per_cu<EK, W, NSUB, SRC, FEAT>() && DPAD * T::CB == 256;
  // otherwise tile j lives in LDS buffer j % 3: tile i is being multiplied
  // (from registers), tile i+1's A fragments are being read, tile i+2 is
  // being written
  constexpr int NBUF = kDMA ? 4 : 3;
  constexpr int TBYTES = kDMA ? 32 * 256 : T::TILE_B;
  __shared__ __attribute__((aligned(16))) char s_tile[NBUF][T::NARR][TBYTES];
  __shared__ __attribute__((aligned(16))) float s_rs[4][32];  // fp8 per-row scale of tile j in slot j % 4
  // Finished documents: per-column maxima (already scaled, 0 for invalid
  // columns) of the last NSLOT docs and their local indices. A half is summed
  // per unit and written out one iteration after it fills. (16 slots; 8 in the
  // DMA kernel, whose fourth tile buffer takes the LDS.)
  constexpr int NSLOT = (kDMA || NSUB > 4) ? 8 : 16;  // 4 x 6: two workgroups per CU need the LDS
  constexpr int HSLOT = NSLOT / 2;
  __shared__ __attribute__((aligned(16))) float s_colb[NSLOT][COLS];
  __shared__ int s_slotk[NSLOT];
  __shared__ float s_bw[SRC == SRC_PLAID ? 256 : 1];
  __shared__ int64_t s_doff[kRMax];  // dense: byte offset of token 0; PLAID: first token index
  __shared__ float* s_outp[COLS];      // per unit of the group: &out[u, jl0] (null: no unit)
  __shared__ int32_t s_dlen[kRMax];  // length | holes << 31
  __shared__ __attribute__((aligned(16))) i32x4 s_nz[kRMax + 1];  // {k, length | holes << 31, start lo, hi}; [nnz] = sentinel
  __shared__ int s_nnz, s_ntiles;
  // Flat tiles (DMA kernel): the tiles are 32-row windows of the range's docs
  // laid end to end, so a doc's last tile is not padded to 32 rows; a doc may
  // end inside a tile and the next one start there. Packed docs (F_CU, rows
  // contiguous in memory) take it when every non-empty doc of the range has
  // at least 16 tokens (two doc ends per tile at most); strided docs when
  // every one has at least 32 (one end per tile; each lane tracks the doc of
  // its row).
  // s_sst[m]: position of non-empty doc m's token 0 in that sequence ([nnz]:
  // the total, [nnz + 1]: INT_MAX); s_rb[m]: byte offset of its token 0 from
  // non-empty doc 0's, minus s_sst[m] row strides (mod 2^32), so the row at
  // position P of doc m is at s_rb[m] + P * row stride.
#ifndef LIK_FLAT_TILES
#define LIK_FLAT_TILES 1
#endif
  constexpr bool kFlatOK = LIK_FLAT_TILES && kDMA && SRC == SRC_DENSE;
  constexpr bool kTwoEnd = (FEAT & F_CU) != 0;  // packed docs: two doc ends per tile
  constexpr int kFlatMinLen = kTwoEnd ? 16 : 32;
  __shared__ int32_t s_sst[kFlatOK ? kRMax + 2 : 1];
  __shared__ uint32_t s_rb[kFlatOK ? kRMax + 1 : 1];
  __shared__ int s_flat;

  const bool f_mask = (FEAT & F_MASK) && p.d.mask != nullptr;
  const bool f_ts = (FEAT & F_TS) && p.d.ts != nullptr;
  // p.normalize: bit 0 normalises query tokens, bit 1 doc tokens
  const bool f_norm_q = (SRC == SRC_PLAID || (FEAT & (F_NORM | F_NORMQ))) && (p.normalize & 1);
  const bool f_norm = (SRC == SRC_PLAID || (FEAT & F_NORM)) && (p.normalize & 2);
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
  // Row scales start at 0 (the first iteration's epilogue runs on the
  // -inf-initialised accumulator set; the epilogue keeps -inf rows at -inf
  // whatever their scale).
  for (int i = tid; i < 4 * 32; i += NT) s_rs[i >> 5][i & 31] = 0.f;

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
  // Holes-only launch of the two-launch mask split (doc_filter 2): a
  // workgroup whose docs all keep prefix masks has nothing to score; it
  // leaves here, before loading its query block (block-uniform decision).
  if constexpr (SRC == SRC_DENSE) {
    if (p.doc_filter == 2) {
      int any = 0;
      for (int64_t k = jl0 + tid; k < jl1; k += NT) {
        const int64_t dg = dglob(k);
        any |= (dg >= 0 && p.holes[dg] != 0) ? 1 : 0;
      }
      if (!__syncthreads_or(any)) return;
    }
  }

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
        if (float* o = s_outp[t]) ((__attribute__((address_space(1))) float*)o)[k * p.osd] = 0.f;
    }
  }
  __syncthreads();
  if (wv == 0) {
    int base = 0, ntl = 0, run = 0;
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
      if constexpr (kFlatOK) {
        // positions of the non-empty docs in the flat sequence (exclusive scan)
        int sc = L;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const int t = __shfl_up(sc, o);
          if (lane >= o) sc += t;
        }
        if (nz) s_sst[pos] = run + sc - L;
        run += __shfl(sc, 63);
      }
    }
    if (lane == 0) {
      s_nnz = base;
      s_ntiles = ntl;
      s_nz[base] = (i32x4){0, 0, 0, 0};  // sentinel: an empty doc past the last one
      if constexpr (kFlatOK) {
        s_sst[base] = run;
        s_sst[base + 1] = 0x7fffffff;
        s_rb[base] = 0u;
      }
    }
  }
  __syncthreads();
  const int nnz = __builtin_amdgcn_readfirstlane(s_nnz);
  if (nnz == 0) return;
  if constexpr (kFlatOK) {
    // flat tiles need every doc >= kFlatMinLen tokens and every
    // row within 4 GiB after non-empty doc 0's first row (32-bit DMA offsets)
    if (wv == 0) {
      const int64_t off0 = (int64_t)(uint32_t)s_nz[0][2] | ((int64_t)s_nz[0][3] << 32);
      const int64_t sl = p.d.sl_b;
      bool ok = true;
      int nshort = 0;  // docs under 32 tokens (tiles that hold two doc ends)
      for (int m = lane; m < nnz; m += 64) {
        const i32x4 e = s_nz[m];
        const int64_t L = e[1] & 0x7fffffff;
        const int64_t rel = ((int64_t)(uint32_t)e[2] | ((int64_t)e[3] << 32)) - off0;
        ok = ok && L >= kFlatMinLen && rel >= 0 && rel + (L - 1) * sl + 256 <= 0xffff0000LL;
        nshort += L < 32 ? 1 : 0;
        s_rb[m] = (uint32_t)rel - (uint32_t)s_sst[m] * (uint32_t)sl;
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) nshort += __shfl_xor(nshort, o);
      const bool all = __ballot(!ok) == 0ull;
      // two-end tiles cost a second split and an early doc end: with many of
      // them (C3's log-uniform lengths: 14% of docs under 32 tokens) per-doc
      // tiles measure faster, so flat tiles need at most 1 in 16 short docs
      if (lane == 0) s_flat = (all && sl > 0 && nshort * 16 <= nnz) ? 1 : 0;
    }
    __syncthreads();
  }
  const bool flat = kFlatOK && __builtin_amdgcn_readfirstlane(s_flat) != 0;
  const int ntiles = flat ? (__builtin_amdgcn_readfirstlane(s_sst[nnz]) + 31) >> 5
                          : __builtin_amdgcn_readfirstlane(s_ntiles);

  // ---------------- query block -> B fragments in VGPRs ----------------
  u32x4 bq[NSUB][KS][FV];
  u32x4 bql[T::SPLIT ? NSUB : 1][T::SPLIT ? KS : 1];
  // Per-column query scale (normalise, fp8 token scales). Padding and masked
  // query columns have zero fragments, so their maxima are 0 (or non-finite,
  // which scores 0) without a scale: kernels with neither feature keep none.
  constexpr bool kQsc = SRC == SRC_PLAID || (FEAT & (F_NORM | F_NORMQ | F_TS)) != 0;
  float qsc[kQsc ? NSUB : 1];
#pragma unroll
  for (int sub = 0; sub < NSUB; ++sub) {
    const int col = (wv * NSUB + sub) * 32 + l32;
    const int ul = col / p.LU;
    const int s = col - ul * p.LU;
    bool valid = ul < p.QPG;
    int64_t q = 0, tok = 0;
    if (p.pair_q) {
      q = p.pair_q[g];
      tok = p.q_tok0 + s;
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
        if (f_norm_q) ss += chunk_sumsq<EK>(raw[c]);
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
    float sc = f_norm_q ? inv_norm(ss) : 1.f;
    if (valid && p.q.ts) sc *= p.q.ts[q * p.q.tsn + tok * p.q.tsl];
    if constexpr (kQsc) qsc[sub] = valid ? sc : 0.f;
  }


  // ---------------- tile cursor and descriptors ----------------
  // One cursor walks the workgroup's tiles in order (tile t of the m-th
  // non-empty doc). Each iteration it emits the descriptor of the newest tile
  // (the one being fetched) and advances: a doc boundary selects the next
  // table entry, and past the last doc the sentinel entry (length 0) makes
  // every further tile empty. Older tiles' descriptors move down a
  // short register queue (fetch -> commit -> MFMA -> epilogue).
  struct Cur {
    int m, t, len, k;
    bool holes;
    int64_t off;  // dense: byte offset of the doc's token 0; PLAID: its first token index
  };
  struct Desc {
    int nv;       // valid rows of the tile (0..32)
    int t;        // tile index within its doc
    int k;        // doc index within the workgroup's range
    bool docend;  // last tile of its doc
    bool holes;   // doc has a mask with holes (dense)
    int64_t tok;  // PLAID: index of the tile's first token
  };
  auto cur_entry = [&](Cur& c, int m) {
    const i32x4 e = s_nz[m];
    const int v = __builtin_amdgcn_readfirstlane(e[1]);
    c.m = m;
    c.t = 0;
    c.k = __builtin_amdgcn_readfirstlane(e[0]);
    c.len = v & 0x7fffffff;
    c.holes = v < 0;
    c.off = (int64_t)(uint32_t)__builtin_amdgcn_readfirstlane(e[2]) |
            ((int64_t)__builtin_amdgcn_readfirstlane(e[3]) << 32);
  };
  auto cur_adv = [&](Cur& c) {
    // the table is read only at a doc's last tile (a uniform branch)
    if ((c.t + 1) * 32 >= c.len)
      cur_entry(c, c.m + 1 < nnz ? c.m + 1 : nnz);
    else
      c.t += 1;
  };
  auto produce = [&](const Cur& c) -> Desc {
    Desc d;
    const int rem = c.len - c.t * 32;  // >= 0: the cursor stops at a doc's end
    d.nv = rem < 32 ? rem : 32;  // (min, not a clamp: a clamp would leave the scalar unit)
    d.k = c.k;
    d.t = c.t;
    d.docend = c.len > 0 && rem <= 32;
    d.holes = c.holes;
    d.tok = c.off + (int64_t)c.t * 32;
    return d;
  };

  // ---------------- staging: fetch (global -> VGPR ring) and commit (-> LDS) ----------------
  // Staging registers of fetched tiles. Two slots (tile i+4 is fetched while
  // tile i+3's data is in flight) unless registers are capped at 256 for two
  // workgroups per CU: then one slot, tile i+3 fetched after tile i+2 is
  // committed (the other workgroup covers the shorter load lead).
  constexpr bool kTwoWg = two_wg_per_cu<EK, W, NSUB, SRC, FEAT>();
  constexpr bool kOneSlot = kTwoWg;
  u32x4 st[kOneSlot ? 1 : 2][NCH][NCV];
  uint32_t sm[SRC == SRC_DENSE ? 2 : 1];          // dense + mask: the tile's row-validity word
  float sts[SRC == SRC_DENSE ? 2 : 1][NCH];       // dense fp8: token scale per row
  uint32_t sb0[SRC == SRC_PLAID ? 2 : 1][NCH];    // PLAID: residual bits (low)
  uint32_t sb1[SRC == SRC_PLAID ? 2 : 1][NCH];    // PLAID: residual bits (high)
  int32_t scode[SRC == SRC_PLAID ? 2 : 1][NCH];   // PLAID: centroid code per row

  // Per-lane constants of the staging chunks: chunk i of this thread is
  // (row, 16-byte column cc) of the tile. lrow is the row, or 64 for chunks
  // that are padding (past the 32 rows or past the embedding dim), so the
  // single test lrow < nv selects the loads that happen. loff is the byte
  // offset of the chunk from the tile's row 0.
  int lrow[NCH];
  uint32_t loff[NCH];
  int lcc[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    // DMA: chunk i of this lane is LDS slot (wave * NCH + i) * 64 + lane of
    // the chunk-major tile, i.e. row slot % 32 and chunk slot / 32
    const int c = kDMA ? (wv * NCH + i) * 64 + lane : tid + i * NT;
    const int row = kDMA ? c % 32 : c / SCPR, cc = kDMA ? c / 32 : c % SCPR;
    const bool inr = FULLCH || c < 32 * SCPR;
    lcc[i] = cc;
    if constexpr (SRC == SRC_DENSE) {
      lrow[i] = (inr && cc * T::CHUNK_E < p.d.dim) ? row : 64;
      loff[i] = (uint32_t)row * (uint32_t)p.d.sl_b + (uint32_t)cc * 16u;
    } else {
      lrow[i] = (inr && cc * 8 < p.q.dim) ? row : 64;
      loff[i] = (uint32_t)row;
    }
  }

  // DMA lane offsets from the tile's row 0 (padding chunks out of range)
  uint32_t dmaoff[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) dmaoff[i] = lrow[i] < 32 ? loff[i] : kOOB;
  // flat tiles: offset of this lane's chunk within its row (kOOB: padding chunk)
  uint32_t dmacc[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) dmacc[i] = lrow[i] < 32 ? (uint32_t)lcc[i] * 16u : kOOB;

  // PLAID phase A: centroid codes of tile d
  auto fetch_codes = [&](auto SS, const Desc& d) {
    if constexpr (SRC == SRC_PLAID) {
      constexpr int S = decltype(SS)::value;
      const __amdgpu_buffer_rsrc_t rc = make_rsrc(p.pl.codes + d.tok, (uint32_t)d.nv * 4u);
#pragma unroll
      for (int i = 0; i < NCH; ++i)
        scode[S][i] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rc, lrow[i] < d.nv ? loff[i] * 4u : kOOB, 0, 0);
    }
  };

  // Dense: token data of the cursor's current tile into slot S (rows past
  // the doc end and padding chunks are out of range and read as 0).
  // DMA fetch of tile d straight into LDS buffer buf (two-workgroup kernel).
  // Issued as inline asm: the compiler treats a DMA write as aliasing every
  // later LDS read and would wait for all DMA before each A-fragment read;
  // here the ordering is explicit (the step-end wait and barrier). M0 (the
  // LDS destination) is saved and restored around the load.
  // The buffer descriptor starts at the tile's first row and ends with its
  // last valid row, so rows past the doc end fall out of range (and read 0)
  // with no per-lane test: the lane offsets are loop constants (dmaoff).
  auto dma_issue = [&](int buf, int i, uint32_t voff, const u32x4& desc) {
    const int wu = __builtin_amdgcn_readfirstlane(wv);
    const uint32_t lds = (uint32_t)__builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)(s_tile[buf][0] + (wu * NCH + i) * 1024));
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"  // an M0 write needs one wait state before an LDS DMA reads it
        "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(lds), "v"(voff), "s"(desc)
        : "memory");
  };
  auto fetch_dma = [&](const Cur& c, const Desc& d, int buf) {
    if constexpr (kDMA) {
      const uint32_t sl = (uint32_t)p.d.sl_b;
      const uint32_t span = d.nv > 0 ? (uint32_t)(d.nv - 1) * sl + (uint32_t)(p.d.dim * T::IN_B) : 0u;
      const uint64_t base = (uint64_t)(p.d.data + c.off) + (uint64_t)((uint32_t)c.t * 32u * sl);
      // raw buffer descriptor: base, stride 0, num_records = span, untyped 32-bit format
      const u32x4 desc = {(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)base),
                          (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(base >> 32) & 0xffffu),
                          (uint32_t)__builtin_amdgcn_readfirstlane(span), 0x00020000u};
#pragma unroll
      for (int i = 0; i < NCH; ++i) dma_issue(buf, i, dmaoff[i], desc);
    }
  };
  // DMA offsets of the flat tile at position P. Lane row l32 of the tile is
  // position P + l32: for packed docs at (P + l32) row strides from non-empty
  // doc 0's first row; else (lm, lE, lb) track the non-empty doc that
  // position is in (its index, end position and s_rb entry): positions
  // advance by 32 per tile and such docs are >= 32 tokens, so a lane crosses
  // at most one doc end per tile. Positions past the last doc read 0 (offset kOOB). The offsets are
  // computed one step ahead of their DMA, which then needs no LDS read or
  // wait and can issue among the tile's MFMAs; the DMA uses the raw
  // descriptor dflat at non-empty doc 0's first row (range 0xfffffff0).
  auto flat_offsets = [&](int P, int& lm, int& lE, uint32_t& lb, int total, uint32_t (&vo)[NCH]) {
    if constexpr (kFlatOK) {
      const int pr = P + l32;
      if constexpr (!kTwoEnd) {
        if (pr >= lE) {
          lm += 1;
          lE = s_sst[lm + 1];
          lb = s_rb[lm];
        }
      }
      const bool live = pr < total;
      const uint32_t roff = (kTwoEnd ? 0u : lb) + (uint32_t)pr * (uint32_t)p.d.sl_b;
#pragma unroll
      for (int i = 0; i < NCH; ++i) vo[i] = (live && dmacc[i] != kOOB) ? roff + dmacc[i] : kOOB;
    }
  };
  auto fetch_dense = [&](auto SS, const Cur& c, const Desc& d) {
    if constexpr (SRC == SRC_DENSE) {
      constexpr int S = kOneSlot ? 0 : decltype(SS)::value;
      // one doc spans < 4 GiB (checked on the host), so 32-bit math is exact
      const uint32_t span = (uint32_t)(c.len > 1 ? c.len - 1 : 0) * (uint32_t)p.d.sl_b + (uint32_t)(p.d.dim * T::IN_B);
      const __amdgpu_buffer_rsrc_t rd = make_rsrc(p.d.data + c.off, span);
      const uint32_t toff = (uint32_t)c.t * 32u * (uint32_t)p.d.sl_b;
#pragma unroll
      for (int i = 0; i < NCH; ++i)
        st[S][i][0] = __builtin_amdgcn_raw_buffer_load_b128(rd, lrow[i] < d.nv ? loff[i] + toff : kOOB, 0, 0);
      if constexpr ((FEAT & (F_MASK | F_TS)) != 0) {
        const int64_t doc = dglob(jl0 + c.k);
        if constexpr ((FEAT & F_MASK) != 0) {
          // validity word of the tile (only docs with mask holes have one)
          const __amdgpu_buffer_rsrc_t rm =
              make_rsrc(p.tbits + (doc >= 0 ? doc : 0) * p.tbits_sn, sat_u32(p.tbits_sn * 4));
          sm[S] = __builtin_amdgcn_raw_buffer_load_b32(rm, (f_mask && c.holes) ? (uint32_t)c.t * 4u : kOOB, 0, 0);
        }
        if constexpr ((FEAT & F_TS) != 0) {
          const __amdgpu_buffer_rsrc_t rt =
              make_rsrc(p.d.ts + (doc >= 0 ? doc : 0) * p.d.tsn, f_ts ? span_bytes(c.len, p.d.tsl, 4) : 0u);
#pragma unroll
          for (int i = 0; i < NCH; ++i) {
            const int64_t tok = (int64_t)c.t * 32 + (lrow[i] & 31);
            sts[S][i] = __uint_as_float(
                __builtin_amdgcn_raw_buffer_load_b32(rt, lrow[i] < d.nv ? sat_u32(tok * p.d.tsl * 4) : kOOB, 0, 0));
          }
        }
      }
    }
  };

  // PLAID phase B: centroid rows (by the codes in slot S) and residual bits of tile d.
  const __amdgpu_buffer_rsrc_t rcent =
      SRC == SRC_PLAID ? make_rsrc(p.pl.cent, sat_u32(p.pl.ncent * p.pl.cent_sb)) : make_rsrc(nullptr, 0u);
  auto fetch_plaid = [&](auto SS, const Desc& d) {
    if constexpr (SRC == SRC_PLAID) {
      constexpr int S = decltype(SS)::value;
      const __amdgpu_buffer_rsrc_t rres =
          make_rsrc(p.pl.res + d.tok * p.pl.res_st, sat_u32((int64_t)d.nv * p.pl.res_st));
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const bool ok = lrow[i] < d.nv;
        int64_t code = scode[S][i];
        code = (code < 0 || code >= p.pl.ncent) ? 0 : code;
        const uint32_t coff = ok ? (uint32_t)(code * p.pl.cent_sb) + (uint32_t)(lcc[i] * 8 * CSZ) : kOOB;
        st[S][i][0] = __builtin_amdgcn_raw_buffer_load_b128(rcent, coff, 0, 0);
        if constexpr (NCV > 1) st[S][i][1] = __builtin_amdgcn_raw_buffer_load_b128(rcent, ok ? coff + 16u : kOOB, 0, 0);
        const uint32_t roff = ok ? loff[i] * (uint32_t)p.pl.res_st + (uint32_t)(lcc[i] * p.pl.nbits) : kOOB;
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

  // fp8 rows cannot be rescaled in place, so an fp8 doc with a per-row scale
  // (token scale or normalise) keeps it in s_rs and the epilogue applies it.
  constexpr bool kRowScaleEpi = SRC == SRC_DENSE && EK == EK_FP8 && (FEAT & (F_TS | F_NORM)) != 0;
  const bool row_scale = kRowScaleEpi && (f_norm || f_ts);

  // Commit the tile staged in VGPR slot S to LDS buffer `buf`: dense
  // bf16/f16/f32 rows are L2-normalised here (scaled in fp32, rounded once
  // to the MFMA type); PLAID rows are decoded, normalised and rounded. Rows
  // past the tile's valid ones are written as zeros.
  auto commit = [&](auto SS, const Desc& d, int buf, int rslot) {
    constexpr int S = kOneSlot ? 0 : decltype(SS)::value;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int row = (tid + i * NT) / SCPR, cc = lcc[i];
      const bool inr = FULLCH || tid + i * NT < 32 * SCPR;
      if constexpr (SRC == SRC_DENSE) {
        float ss = 0.f;
        if (f_norm) {
          ss = chunk_sumsq<EK>(st[S][i][0]);
#pragma unroll
          for (int o = 1; o < SCPR; o <<= 1) ss += __shfl_xor(ss, o);
        }
        u32x4 v = st[S][i][0];
        if constexpr (EK != EK_FP8) {
          if (f_norm) {
            const float sc = inv_norm(ss);
            if constexpr (EK == EK_BF16) {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                v[e] = f32_to_bf16_bits(bf16lo_to_f32(v[e]) * sc) | (f32_to_bf16_bits(bf16hi_to_f32(v[e]) * sc) << 16);
            } else if constexpr (EK == EK_F16) {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                v[e] = f32_to_f16_bits(f16_to_f32((uint16_t)(v[e] & 0xffffu)) * sc) |
                       (f32_to_f16_bits(f16_to_f32((uint16_t)(v[e] >> 16)) * sc) << 16);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e) v[e] = __float_as_uint(__uint_as_float(v[e]) * sc);
            }
          }
        }
        if constexpr ((FEAT & F_MASK) != 0) {
          // rows the mask drops are written as zeros: their -inf bias then
          // gives -inf whatever the row held (a NaN or inf there would
          // otherwise turn -inf + x into NaN and poison the max)
          if (d.holes && !((sm[S] >> (row & 31)) & 1u)) v = (u32x4){0u, 0u, 0u, 0u};
        }
        if (inr) {
          char* rowp = s_tile[buf][0] + row * T::ROW_B;
          if constexpr (T::SPLIT) {
            u32x2 hi, lo;
            split4(v, hi, lo);
            *(u32x2*)(rowp + cc * 8) = hi;
            *(u32x2*)(s_tile[buf][1] + row * T::ROW_B + cc * 8) = lo;
          } else {
            *(u32x4*)(rowp + cc * 16) = v;
          }
          if constexpr (kRowScaleEpi) {
            if (cc == 0) s_rs[rslot][row] = (f_norm ? inv_norm(ss) : 1.f) * (f_ts ? sts[S][i] : 1.f);
          }
        }
      } else {
        (void)rslot;
        const bool live = row < d.nv;
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
        const float sc = (p.normalize & 2) ? inv_norm(ss) : 1.f;
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
  // Accumulators: set P holds tile i (MFMA in flight), set 1-P holds tile i-1
  // (epilogue), so one wave overlaps tile i's MFMAs with tile i-1's max.
  // Two accumulator sets unless they do not fit in 256 registers next to the
  // query fragments (4 blocks per wave with two waves per SIMD): then one
  // set, the epilogue runs before the tile's MFMAs and the SIMD's other
  // wave covers the gap.
  constexpr int NACC = ((W == 8 && NSUB >= 4) || kTwoWg) ? 1 : 2;
  // Row masking. With two sets it is folded into the MFMA C operand: the
  // first k-step of a tile adds `bias` (0 for valid rows, -inf for rows past
  // the doc end or dropped by the mask), so the epilogue is a plain running
  // max. In the 256-register two-workgroup kernel the 16 bias registers do
  // not fit: tiles start from 0 and the epilogue sets invalid rows to -inf,
  // in partial tiles only.
  constexpr bool kBiasC = !kTwoWg;
  f32x16 acc[NACC][NSUB];
  float m[NSUB];
  int mi[NSUB];  // F_ARGMAX: doc-token index of m (-1: no valid token yet)
#pragma unroll
  for (int sub = 0; sub < NSUB; ++sub) {
    m[sub] = NEG_INF;
    mi[sub] = -1;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[NACC - 1][sub][e] = NEG_INF;
  }
  f32x16 bias;
#pragma unroll
  for (int e = 0; e < 16; ++e) bias[e] = 0.f;
  uint32_t bias_bits = 0xffffffffu;
  uint32_t vb_cur = 0xffffffffu, vb_prev = 0xffffffffu;  // row-valid bits of tiles i, i-1 (no bias)
  // accumulator element e of lane (h, l32) is doc row 8*(e/4) + 4*h + e%4
  auto set_bias = [&](uint32_t vb) {
#pragma unroll
    for (int e = 0; e < 16; ++e) bias[e] = ((vb >> (8 * (e >> 2) + 4 * h + (e & 3))) & 1u) ? 0.f : NEG_INF;
    bias_bits = vb;
  };

  // A fragments (this lane's doc row, both k-halves) of a tile, read from
  // LDS one iteration ahead of their MFMAs into register set S. For large
  // embedding dims the two sets would not fit next to the query fragments,
  // so the MFMA loop reads them from the tile's LDS buffer instead.
  constexpr bool kPrefetchA = KS * FV <= 8 && !kTwoWg;
  u32x4 af[kPrefetchA ? 2 : 1][KS][FV];
  u32x4 afl[kPrefetchA ? 2 : 1][T::SPLIT ? KS : 1];
  auto load_a = [&](auto SS, int buf) {
    constexpr int S = kPrefetchA ? decltype(SS)::value : 0;
    const char* A = s_tile[buf][0] + l32 * T::ROW_B + h * T::HALF_B;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int v = 0; v < FV; ++v) af[S][ks][v] = *(const u32x4*)(A + ks * T::FRAG_B + v * 16);
      if constexpr (T::SPLIT)
        afl[S][ks] = *(const u32x4*)(s_tile[buf][1] + l32 * T::ROW_B + h * T::HALF_B + ks * T::FRAG_B);
    }
  };
  auto mma_tile = [&](auto PP, auto SS, int buf) {
    constexpr int P = NACC == 2 ? decltype(PP)::value : 0;
    constexpr int S = kPrefetchA ? decltype(SS)::value : 0;
    const char* A = s_tile[buf][0] + l32 * T::ROW_B + h * T::HALF_B;
    if constexpr (kTwoWg) {
      // A fragments from LDS inside the tile, two k-steps ahead of their
      // MFMAs (three rotating registers). The fences keep LDS reads and
      // MFMAs in this order and let other instructions move across them.
      constexpr int kFence = 0x2 | 0x4 | 0x10 | 0x20 | 0x40 | 0x200 | 0x400;
      // A fragment k-step ks of this lane: bytes [(h * KS + ks) * FRAG_B, +FRAG_B)
      // of row l32. DMA tiles are chunk-major (16-byte chunk j of row r at
      // j * 512 + r * 16): a fragment's rows are contiguous, so the reads are
      // conflict-free and every (k-step, chunk) offset is an immediate.
      const char* AD = s_tile[buf][0] + h * (KS * FV * 512) + l32 * 16;
      u32x4 a3[3][FV];
      auto lda = [&](int slot, int ks) {
#pragma unroll
        for (int v = 0; v < FV; ++v)
          a3[slot][v] = kDMA ? *(const u32x4*)(AD + (ks * FV + v) * 512) : ((const u32x4*)(A + ks * T::FRAG_B))[v];
      };
      lda(0, 0);
      if constexpr (KS > 1) lda(1, 1);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (ks + 2 < KS) lda((ks + 2) % 3, ks + 2);
        __builtin_amdgcn_sched_barrier(kFence);
#pragma unroll
        for (int sub = 0; sub < NSUB; ++sub)
          acc[P][sub] = mfma32<EK>(ks == 0 ? f32x16{} : acc[P][sub], a3[ks % 3], bq[sub][ks]);
        __builtin_amdgcn_sched_barrier(kFence);
      }
      return;
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if constexpr (!kPrefetchA) {
#pragma unroll
        for (int v = 0; v < FV; ++v) af[0][ks][v] = *(const u32x4*)(A + ks * T::FRAG_B + v * 16);
        if constexpr (T::SPLIT)
          afl[0][ks] = *(const u32x4*)(s_tile[buf][1] + l32 * T::ROW_B + h * T::HALF_B + ks * T::FRAG_B);
      }
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub) {
        f32x16 c = ks == 0 ? (kBiasC ? bias : f32x16{}) : acc[P][sub];
        c = mfma32<EK>(c, af[S][ks], bq[sub][ks]);
        if constexpr (T::SPLIT) {
          c = mfma32<EK>(c, af[S][ks], &bql[sub][ks]);
          c = mfma32<EK>(c, &afl[S][ks], bq[sub][ks]);
        }
        acc[P][sub] = c;
      }
    }
  };

  int nend = 0;  // documents finished so far
  // score scale: out_scale times the per-tensor scales read from device
  // memory (fp8 per-tensor dequant scales, no host read)
  const float osc = p.out_scale * (p.scale_q ? *p.scale_q : 1.f) * (p.scale_d ? *p.scale_d : 1.f);

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
      // global (not generic) store: a flat store would also count in the LDS
      // wait counter and force full waits on the A-fragment reads. (The slot's
      // doc index is checked against the range: a slot the ring logic never
      // filled must not turn into a store outside the output.)
      const int kd = s_slotk[sl];
      if ((unsigned)kd >= (unsigned)nloc) continue;
      auto* o = &((__attribute__((address_space(1))) float*)orow)[kd * p.osd];
      *o = p.accumulate ? sum * osc + *o : sum * osc;
    }
  };

  // Running max over the rows of the previous tile (accumulator set P),
  // whose first row is doc token `row0`.
  auto epilogue = [&](auto PP, int rslot, int row0) {
    constexpr int P = NACC == 2 ? decltype(PP)::value : 0;
    if constexpr (!kBiasC) {
      // rows of tile i-1 that are not valid: -inf before the max
      if (vb_prev != 0xffffffffu) {
        const uint32_t vh = vb_prev >> (4 * h);
#pragma unroll
        for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if (!((vh >> (8 * (e >> 2) + (e & 3))) & 1u)) acc[P][sub][e] = NEG_INF;
      }
    }
    if constexpr ((FEAT & F_ARGMAX) != 0) {
      // rows are visited in increasing index order and only a strictly larger
      // value replaces the winner: ties keep the lowest doc-token index
      const int r0 = row0 + 4 * h;
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float v = acc[P][sub][4 * j + e];
            mi[sub] = v > m[sub] ? r0 + 8 * j + e : mi[sub];
            m[sub] = max_nan(m[sub], v);  // a NaN row makes the max NaN (scored 0, argmax -1)
          }
      (void)rslot;
      return;
    }
    if constexpr (kRowScaleEpi) {
      if (row_scale) {
        f32x4 sc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) sc[j] = *(const f32x4*)&s_rs[rslot][8 * j + 4 * h];
#pragma unroll
        for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              // invalid rows hold -inf and may have a 0 or NaN scale: they stay -inf
              const float a = acc[P][sub][4 * j + e];
              m[sub] = max_nan(m[sub], a == NEG_INF ? NEG_INF : a * sc[j][e]);
            }
        return;
      }
    }
    (void)rslot;
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
      for (int e = 0; e < 16; ++e) m[sub] = max_nan(m[sub], acc[P][sub][e]);
  };

  // The previous tile was the last of doc k: park the per-column maxima.
  auto doc_end = [&](int k) {
    const int sl = nend % NSLOT;
    if constexpr ((FEAT & F_ARGMAX) != 0) {
      // winner over lanes l, l^32 (larger value; equal values: lower index),
      // written to argmax[(q * docs + j) * Lq + token] (pair mode: unit g is
      // the pair, one doc: argmax[pair * Lq + token])
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub) {
        const auto sv = __builtin_amdgcn_permlane32_swap(__float_as_uint(m[sub]), __float_as_uint(m[sub]), false, false);
        const auto si = __builtin_amdgcn_permlane32_swap((uint32_t)mi[sub], (uint32_t)mi[sub], false, false);
        const float v0 = __uint_as_float(sv[0]), v1 = __uint_as_float(sv[1]);
        const int i0 = (int)si[0], i1 = (int)si[1];
        const bool take1 = v1 > v0 || (v1 == v0 && (unsigned)i1 < (unsigned)i0);
        const int win = take1 ? i1 : i0;
        const int col = (wv * NSUB + sub) * 32 + l32;
        const int ul = col / p.LU;
        if (h == 0 && p.amax && ul < p.QPG) {
          const int64_t u = g * p.QPG + ul;
          const int64_t q = u / p.nc;
          const int64_t tok = p.q_tok0 + (u - q * p.nc) * p.LU + (col - ul * p.LU);
          if (u < p.nunits && tok < p.amax_ld)
            p.amax[(q * p.amax_qs + jl0 + k) * p.amax_ld + tok] = __builtin_isfinite(max_nan(v0, v1)) ? win : -1;
        }
        mi[sub] = -1;
      }
    }
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub) {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(m[sub]), __float_as_uint(m[sub]), false, false);
      const float mm = max_nan(__uint_as_float(sw[0]), __uint_as_float(sw[1]));  // max over lanes l, l^32
      if (h == 0) s_colb[sl][(wv * NSUB + sub) * 32 + l32] = __builtin_isfinite(mm) ? (kQsc ? mm * qsc[kQsc ? sub : 0] : mm) : 0.f;
      m[sub] = NEG_INF;
    }
    if (tid == 0) s_slotk[sl] = k;
    ++nend;
  };

  // Flat tiles (one accumulator set): rows [0, b) of tile d end non-empty doc
  // d.k when b = d.nv <= 32, and rows [b, 32) are the first rows of the next
  // one (none past the last doc): their max goes to mn, the next doc's
  // running max once doc d.k is parked. Accumulator element 4 j + r of lane
  // half h is row 8 j + 4 h + r, so for b < 32 only the element group
  // js = b / 8 straddles the boundary (element r below it when
  // r < b - 8 js - 4 h); the groups before it go whole to m, those after it
  // whole to mn, and js is uniform: one unrolled body per value.
  // Packed docs: when the next doc ends in the tile too (at row d.t > 0, a doc
  // shorter than 32 tokens), doc d.k is parked here, its rows are set to
  // -inf, and the same split at d.t gives the next doc's max (m) and the rows
  // after it (mn); the caller then parks doc d.k + 1.
  auto split_at = [&](int b, float (&mn)[NSUB]) {
    const int js = b < 32 ? b >> 3 : 3;  // (b = 32: everything below, through group 3)
    const int ch = b - 8 * js - 4 * h;
    bool lo[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) lo[r] = r < ch;
    auto split = [&](auto JS) {
      constexpr int J = decltype(JS)::value;
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub) {
        float a = m[sub], c = NEG_INF;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float x[4] = {acc[0][sub][4 * j], acc[0][sub][4 * j + 1], acc[0][sub][4 * j + 2], acc[0][sub][4 * j + 3]};
          if (j < J) {
            a = max_nan(a, max_nan(x[0], x[1]));
            a = max_nan(a, max_nan(x[2], x[3]));
          } else if (j > J) {
            c = max_nan(c, max_nan(x[0], x[1]));
            c = max_nan(c, max_nan(x[2], x[3]));
          } else {
            float lv[4], hv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              lv[r] = lo[r] ? x[r] : NEG_INF;
              hv[r] = lo[r] ? NEG_INF : x[r];
            }
            a = max_nan(a, max_nan(lv[0], lv[1]));
            a = max_nan(a, max_nan(lv[2], lv[3]));
            c = max_nan(c, max_nan(hv[0], hv[1]));
            c = max_nan(c, max_nan(hv[2], hv[3]));
          }
        }
        m[sub] = a;
        mn[sub] = c;
      }
    };
    switch (js) {
      case 0: split(std::integral_constant<int, 0>{}); break;
      case 1: split(std::integral_constant<int, 1>{}); break;
      case 2: split(std::integral_constant<int, 2>{}); break;
      default: split(std::integral_constant<int, 3>{}); break;
    }
  };
  auto epilogue_flat = [&](const Desc& d, float (&mn)[NSUB]) {
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub) mn[sub] = NEG_INF;
    if (kTwoEnd && d.docend && d.t > 0) {
      split_at(d.nv, mn);  // m: doc d.k complete (mn unused)
      doc_end(__builtin_amdgcn_readfirstlane(s_nz[d.k][0]));  // (the caller checks the slot ring)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const bool lo = 8 * (e >> 2) + 4 * h + (e & 3) < d.nv;
#pragma unroll
        for (int sub = 0; sub < NSUB; ++sub) acc[0][sub][e] = lo ? NEG_INF : acc[0][sub][e];
      }
      split_at(d.t, mn);  // m: doc d.k + 1 complete, mn: the rows after it
      if (d.k + 2 >= nnz) {
#pragma unroll
        for (int sub = 0; sub < NSUB; ++sub) mn[sub] = NEG_INF;
      }
      return;
    }
    if (!d.docend || d.nv >= 32) {
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
        for (int e = 0; e < 16; ++e) m[sub] = max_nan(m[sub], acc[0][sub][e]);
      return;
    }
    split_at(d.nv, mn);
    if (d.k + 1 >= nnz) {
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub) mn[sub] = NEG_INF;
    }
  };

  // ---------------- prologue ----------------
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  // Pipeline at iteration i: MFMA tile i (A fragments already in registers),
  // read tile i+1's A fragments from LDS, max of tile i-1, commit tile i+2 to
  // LDS, fetch tile i+4 (PLAID: data of tile i+4, codes of tile i+5; one
  // staging slot: tile i+3).
  // Descriptor queue: qm1 = tile i-1, q0 = i, q1 = i+1, q2 = i+2, q3 = i+3
  // (PLAID also q4 = i+4); the cursor produces the newest tile.
  auto run = [&](auto FL) {
  constexpr bool FLAT = decltype(FL)::value;
  Cur cur;
  cur_entry(cur, 0);
  // flat tiles: cursor (position of the newest tile, non-empty doc holding
  // its row 0, that doc's end position) and the lanes' row cursors
  int fP = 0, fm = 0, fend = 0, fend2 = 0, lm = 0, lE = 0, total = 0;
  uint32_t lb = 0u, fvo[NCH];
  u32x4 dflat = {0u, 0u, 0u, 0u};
  if constexpr (FLAT) {
    fend = __builtin_amdgcn_readfirstlane(s_sst[1]);
    fend2 = __builtin_amdgcn_readfirstlane(s_sst[nnz >= 1 ? 2 : 1]);
    lE = s_sst[1];
    lb = s_rb[0];
    total = __builtin_amdgcn_readfirstlane(s_sst[nnz]);
    const uint64_t base = (uint64_t)(p.d.data + ((int64_t)(uint32_t)s_nz[0][2] | ((int64_t)s_nz[0][3] << 32)));
    dflat = u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)base),
                  (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(base >> 32) & 0xffffu), 0xfffffff0u, 0x00020000u};
  }
  // (fend, fend2: end positions of docs fm and fm + 1; s_sst[nnz + 1] is INT_MAX)
  auto fproduce = [&]() -> Desc {
    Desc d{};
    d.k = fm;
    d.nv = fend - fP;  // rows of doc fm from the tile's row 0 (<= 32: it ends in the tile)
    d.docend = fm < nnz && d.nv <= 32;
    // the next doc ends in the tile too (at row d.t)
    d.t = (kTwoEnd && d.docend && d.nv < 32 && fm + 1 < nnz && fend2 - fP <= 32) ? fend2 - fP : 0;
    return d;
  };
  auto fadv = [&]() {
    fP += 32;
#pragma unroll
    for (int x = 0; x < (kTwoEnd ? 2 : 1); ++x) {
      if (fend <= fP) {
        fm += 1;
        fend = fend2;
        fend2 = __builtin_amdgcn_readfirstlane(s_sst[fm + 2 <= nnz + 1 ? fm + 2 : nnz + 1]);
      }
    }
  };
  float mnext[NSUB];
#pragma unroll
  for (int sub = 0; sub < NSUB; ++sub) mnext[sub] = NEG_INF;
  Desc qm1{}, q0, q1, q2, q3, q4{};
  // mask words of tiles i, i+1, i+2 (dense + mask; taken from the staged loads at commit)
  uint32_t vw0 = 0xffffffffu, vw1 = 0xffffffffu, vw2 = 0xffffffffu;
  q0 = FLAT ? fproduce() : produce(cur);
  if constexpr (FLAT) {
    auto pro = [&](int t) {
      flat_offsets(fP, lm, lE, lb, total, fvo);
#pragma unroll
      for (int c = 0; c < NCH; ++c) dma_issue(t, c, fvo[c], dflat);
      fadv();
    };
    pro(0);
    q1 = fproduce();
    pro(1);
    q2 = fproduce();
    pro(2);
    flat_offsets(fP, lm, lE, lb, total, fvo);  // tile 3, issued in step 0
    asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  } else if constexpr (SRC == SRC_DENSE && kDMA) {
    // tiles 0, 1, 2 into buffers 0, 1, 2; the cursor runs three tiles ahead
    // of the MFMA
    fetch_dma(cur, q0, 0);
    cur_adv(cur);
    q1 = produce(cur);
    fetch_dma(cur, q1, 1);
    cur_adv(cur);
    q2 = produce(cur);
    fetch_dma(cur, q2, 2);
    cur_adv(cur);
    // tile 0 landed before the barrier (tiles 1 and 2, 2 * NCH younger
    // instructions, may still be in flight: the first step's end waits)
    asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  } else if constexpr (SRC == SRC_DENSE && kOneSlot) {
    // one staging slot: tiles 0 and 1 committed, tile 2 in flight (the
    // cursor runs three tiles ahead of the MFMA)
    fetch_dense(I0{}, cur, q0);
    cur_adv(cur);
    commit(I0{}, q0, 0, 0);
    q1 = produce(cur);
    fetch_dense(I0{}, cur, q1);
    cur_adv(cur);
    commit(I0{}, q1, 1, 1);
    q2 = produce(cur);
    fetch_dense(I0{}, cur, q2);
    cur_adv(cur);
  } else if constexpr (SRC == SRC_DENSE) {
    fetch_dense(I0{}, cur, q0);
    cur_adv(cur);
    q1 = produce(cur);
    fetch_dense(I1{}, cur, q1);
    cur_adv(cur);
    commit(I0{}, q0, 0, 0);
    if constexpr ((FEAT & F_MASK) != 0) vw0 = sm[0];
    q2 = produce(cur);
    fetch_dense(I0{}, cur, q2);
    cur_adv(cur);
    commit(I1{}, q1, 1, 1);
    if constexpr ((FEAT & F_MASK) != 0) vw1 = sm[1];
    q3 = produce(cur);
    fetch_dense(I1{}, cur, q3);
    cur_adv(cur);
  } else {
    fetch_codes(I0{}, q0);
    cur_adv(cur);
    q1 = produce(cur);
    fetch_codes(I1{}, q1);
    cur_adv(cur);
    fetch_plaid(I0{}, q0);
    fetch_plaid(I1{}, q1);
    q2 = produce(cur);
    fetch_codes(I0{}, q2);
    cur_adv(cur);
    commit(I0{}, q0, 0, 0);
    fetch_plaid(I0{}, q2);
    q3 = produce(cur);
    fetch_codes(I1{}, q3);
    cur_adv(cur);
    commit(I1{}, q1, 1, 1);
    fetch_plaid(I1{}, q3);
    q4 = produce(cur);
    fetch_codes(I0{}, q4);
    cur_adv(cur);
  }
  __syncthreads();
  if constexpr (kPrefetchA) load_a(I0{}, 0);
  int buf_x = 0;          // LDS buffer of tile i
  int buf_a = 1;          // LDS buffer of tile i+1
  int buf_c = 2;          // LDS buffer of tile i+2
  int flush_half = -1;    // slot half whose flush is due (after the barrier it waited for)

  // ---------------- main loop (unrolled by 2 so register slots are static) ----------------
  auto step = [&](auto PP, int i) {
    constexpr int P = decltype(PP)::value;
    using IP = std::integral_constant<int, P>;
    using IQ = std::integral_constant<int, 1 - P>;
    if (flush_half >= 0) {
      flush(flush_half * HSLOT, HSLOT);
      flush_half = -1;
    }
    if constexpr (!FLAT) {
      // row validity of tile i (uniform): rows past the doc end, and rows the
      // mask drops in docs with holes
      uint32_t vb = q0.nv >= 32 ? 0xffffffffu : ((1u << q0.nv) - 1u);
      if constexpr (SRC == SRC_DENSE && (FEAT & F_MASK) != 0) {
        if (q0.holes) vb &= vw0;
      }
      vb = __builtin_amdgcn_readfirstlane(vb);
      if constexpr (kBiasC) {
        if (vb != bias_bits) set_bias(vb);
      } else {
        vb_prev = vb_cur;
        vb_cur = vb;
      }
    }
    // one block: MFMA tile i, read A of tile i+1, max of tile i-1, commit
    // tile i+2, fetch tile i+4
    const Desc qn = FLAT ? fproduce() : produce(cur);
    const int bx = kDMA ? (i & 3) : buf_x;
    if constexpr (NACC == 2) {
      mma_tile(IP{}, IP{}, bx);
      epilogue(IQ{}, (i + 3) & 3, qm1.t * 32);
    } else {
      if constexpr (FLAT) {
        epilogue_flat(qm1, mnext);
        if (kTwoEnd && qm1.docend && qm1.t > 0 && (nend % HSLOT) == 0) flush_half = ((nend / HSLOT) - 1) & 1;
      } else {
        epilogue(IQ{}, (i + 3) & 3, qm1.t * 32);
      }
      mma_tile(IP{}, IP{}, bx);
      // the max stays with the MFMAs that overwrite its accumulators (sunk
      // below the branches that follow, it would keep two sets live)
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub) asm volatile("" : "+v"(m[sub]));
    }
    if constexpr (kPrefetchA) load_a(IQ{}, buf_a);
    if constexpr (!kDMA) commit(IP{}, q2, buf_c, (i + 2) & 3);
    if constexpr (SRC == SRC_DENSE && (FEAT & F_MASK) != 0) vw2 = sm[P];
    if constexpr (FLAT) {
#pragma unroll
      for (int c = 0; c < NCH; ++c) dma_issue((i + 3) & 3, c, fvo[c], dflat);
    } else if constexpr (SRC == SRC_DENSE && kDMA) {
      fetch_dma(cur, qn, (i + 3) & 3);  // tile i+3 straight into its LDS buffer
    } else if constexpr (SRC == SRC_DENSE) {
      fetch_dense(IP{}, cur, qn);  // tile i+4 into slot (i+4)%2 (one slot: tile i+3, after the commit)
    } else {
      fetch_plaid(IP{}, q4);       // tile i+4, codes from slot (i+4)%2
      fetch_codes(IQ{}, qn);       // codes of tile i+5 into slot (i+5)%2
    }
    if constexpr (FLAT) {
      fadv();
      flat_offsets(fP, lm, lE, lb, total, fvo);  // the next step's tile
    } else {
      cur_adv(cur);
    }
    if constexpr (SRC == SRC_DENSE && NACC == 2) {
      // Interleave the block: each MFMA is followed by a few VALU / SALU
      // instructions (epilogue max, commit, fetch addressing, cursor), an LDS
      // read (next tile's A fragments) and a buffer load, so one wave keeps
      // the matrix core fed while it does the tile bookkeeping. The commit's
      // LDS write goes near the end, so its wait for the staged data (loaded
      // two iterations earlier) comes as late as possible.
      constexpr int NM = KS * NSUB * (T::SPLIT ? 3 : 1);
#pragma unroll
      for (int k = 0; k < NM; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // VALU
        __builtin_amdgcn_sched_group_barrier(0x004, 2, 0);  // SALU
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
        if (k == NM - 3) __builtin_amdgcn_sched_group_barrier(0x200, 4 * NCH, 0);  // DS write
      }
    }
    if (i >= 1 && qm1.docend) {
      if constexpr (FLAT) {
        // (a tile with two doc ends parked the first in its epilogue; two
        // ends in one step cross at most one half of the slot ring)
        doc_end(__builtin_amdgcn_readfirstlane(s_nz[qm1.k + (qm1.t > 0 ? 1 : 0)][0]));
#pragma unroll
        for (int sub = 0; sub < NSUB; ++sub) m[sub] = mnext[sub];
      } else {
        doc_end(qm1.k);
      }
      if ((nend % HSLOT) == 0) flush_half = ((nend / HSLOT) - 1) & 1;
    }
    qm1 = q0;
    q0 = q1;
    q1 = q2;
    if constexpr (SRC == SRC_DENSE && kOneSlot) {
      q2 = qn;
    } else if constexpr (SRC == SRC_DENSE) {
      q2 = q3;
      q3 = qn;
    } else {
      q2 = q3;
      q3 = q4;
      q4 = qn;
    }
    vw0 = vw1;
    vw1 = vw2;
    buf_x = buf_a;
    buf_a = buf_a == 2 ? 0 : buf_a + 1;
    buf_c = buf_c == 2 ? 0 : buf_c + 1;
    if constexpr (kDMA) {
      // Tile i+1 must have landed before any wave reads it: this wave's DMA
      // of tile i+1 is older than those of tiles i+2 and i+3 (2 * NCH
      // instructions), and loads complete in order. The barrier has no
      // memory fence (a fence would wait for all DMA); the clobber keeps the
      // compiler from moving LDS accesses across it.
      static_assert(NCH == 2, "vmcnt below assumes 2 DMA instructions per wave and tile");
      asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    } else {
      __syncthreads();
    }
  };
  // iterations 0..ntiles: iteration ntiles only finishes tile ntiles-1 (its
  // MFMA, commit and fetch work on empty tiles and are discarded)
  for (int i = 0;; i += 2) {
    step(I0{}, i);
    if (i + 1 > ntiles) break;
    step(I1{}, i + 1);
    if (i + 2 > ntiles) break;
  }
  // remaining finished docs: the due half (if any) and the partial half
  if (flush_half >= 0) flush(flush_half * HSLOT, HSLOT);
  if (nend % HSLOT) flush(nend - nend % HSLOT, nend % HSLOT);
  };
  if constexpr (kFlatOK) {
    if (flat)
      run(std::true_type{});
    else
      run(std::false_type{});
  } else {
    run(std::false_type{});
  }
  // no DMA may still be writing this workgroup's LDS when it exits
  if constexpr (kDMA) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}
template <int EK, int DPAD, int W, int NSUB, int SRC, int CD, int FEAT>
int launch_one(const Params& p, int64_t nblocks, hipStream_t s) {
  if constexpr (!cfg_ok<EK, DPAD, NSUB>()) {
    return LIK_ERR_UNSUPPORTED;
  } else {
    if (nblocks <= 0) return LIK_OK;
    if (nblocks > 0x7fffffffLL) return LIK_ERR_UNSUPPORTED;
    launch_kernel(maxsim_kernel<EK, DPAD, W, NSUB, SRC, CD, FEAT>, dim3((unsigned)nblocks), dim3(W * 64), 0, s, p);
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
  // fp8 4 x 6: every feature set, since one call may add a masked launch
  if constexpr (EK == EK_FP8 && DPAD <= 128 && SRC == SRC_DENSE)
    if (pl.W == 4 && pl.NSUB == 6) return launch_one<EK, DPAD, 4, 6, SRC, CD, FEAT>(p, nb, s);
  if (pl.W == 8 && pl.NSUB == 1) return launch_one<EK, DPAD, 8, 1, SRC, CD, FEAT>(p, nb, s);
  if (pl.W == 8 && pl.NSUB == 2) return launch_one<EK, DPAD, 8, 2, SRC, CD, FEAT>(p, nb, s);
  if (pl.W == 8 && pl.NSUB == 4) return launch_one<EK, DPAD, 8, 4, SRC, CD, FEAT>(p, nb, s);
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
  return (p.d.mask ? F_MASK : 0) | ((p.d.ts || p.q.ts) ? F_TS : 0) |
         ((p.normalize & 2) ? F_NORM : (p.normalize & 1) ? F_NORMQ : 0) | (p.d.cu ? F_CU : 0);
}

}  // namespace lik
