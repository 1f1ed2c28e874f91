// PLAID residual MaxSim for a few queries over a prepared corpus (gfx950):
// scores from centroid scores instead of centroid rows.
//
// A decoded token is x = c + r: c its centroid row, r the bucket weights
// picked by its residual fields. With the token's inverse norm known ahead
// (lik_plaid_token_records / lik_plaid_token_norms, once per corpus), the
// normalised score of query
// token s is
//     q_s . x / ||x|| = (q_s . c + q_s . r) / ||x||.
// q_s . c depends on the centroid alone, so for each query it is one
// [n_centroids, 32] table (centroid_scores_kernel: 32 centroids x 32 query
// tokens per MFMA tile, times the query token's inverse norm, stored as
// fp16, 64 bytes per centroid), computed per call in a few microseconds.
// The scan then needs, per token, its code, residual bytes and inverse norm
// (40 B at d = 128, nbits = 2) from HBM and one 64-byte table row from L2,
// instead of a 256-byte centroid row: 4x fewer gathered bytes, and no
// per-element decode or norm arithmetic in the loop. q_s . r stays on the
// MFMA (residual fields -> bucket weights rounded to the MFMA type, one
// 32x32 tile product per 32 tokens, as in the split-form gather kernel).
//
// Per wavefront: one (query group, doc range). The range's tokens are one
// contiguous slice of the packed corpus (cu_seqlens layout), walked in flat
// 32-token tiles that ignore doc boundaries, so stream addresses simply
// advance by a tile per iteration; the doc whose tokens continue into the
// tile is tracked by its end token, and a tile holding a doc end is reduced
// segment by segment. Everything a tile needs arrives in LDS by buffer_load ... lds (M0
// saved and restored): the table rows of its tokens (gathered by code, row R
// at position R ^ ((R / 4) % 2) so the two rows one fragment read touches
// sit in different banks), its residual bytes and inverse norms (streaming,
// non-temporal, so they do not push the table out of L2), and, two tiles
// earlier, its codes. Two stages per wave: while tile c is scored from one,
// tile c + 1 lands in the other, and tile c + 2's gather is issued as soon
// as tile c has been read into registers. All of these are loads, which
// return in issue order, so one fixed vmcnt per iteration waits for exactly
// the tile about to be scored. Nothing else in the loop touches vector
// memory: the doc boundaries are staged in LDS and doc scores are collected
// in LDS and written after the loop (a compiler-visible vector memory access
// in the loop would bring a full vmcnt(0) with it). The tile is scored as
//     v[t][s] = (acc[t][s] * qsc[s] + qc[code_t][s]) * inv_t
// (acc = the q . r MFMA, the fp16 table value added by v_fma_mix), a running
// max per column over each doc's rows, and at a doc's end the column maxima
// are summed in the tile kernel's order.
//
// Reference semantics: plaid.py:684-963 / reference.py:142-179 (decode,
// normalise, MaxSim); out-of-range codes decode as centroid 0, out-of-range
// bucket codes as the last bucket.
#include "lik_kernel.h"

namespace lik {

constexpr int kQcRMax = 128;  // docs per wavefront of the scan (host caps R)

// qc[q * qc_qs + c * 32 + s] = fp16(qsc_s * (q_s . c)), for every centroid c
// and the 32 token slots of query q (0 past its length). One wavefront per
// (query, 32 centroids).
// perm: query token s at slot 16 ((s >> 2) & 1) + 4 (s >> 3) + (s & 3) of the
// row (the element order of plaid_scan_kernel's accumulators), else at slot s.
template <int EK, int DPAD>
__global__ void __launch_bounds__(256) centroid_scores_kernel(const Params p, uint16_t* __restrict__ qc,
                                                              int64_t qc_qs, int64_t ntile, int perm) {
  using T = KT<EK, DPAD>;
  constexpr int KS = T::KSTEPS;
  constexpr int HALF = DPAD / 2;
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t q = w / ntile, tile = w - q * ntile;
  if (q >= p.q.n) return;
  const bool valid = l32 < seq_len(p.q, q);
  const char* qrow = valid ? seq_row0(p.q, q) + (int64_t)l32 * p.q.sl_b : nullptr;
  const int64_t c = tile * 32 + l32;
  const bool cvalid = c < p.pl.ncent;
  const char* crow = p.pl.cent + (cvalid ? c : 0) * p.pl.cent_sb;
  float ss = 0.f;
  f32x16 acc = {};
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int e = h * HALF + ks * 8;
    const u32x4 b = (valid && e < p.q.dim) ? *(const u32x4*)(qrow + (int64_t)e * 2) : (u32x4){0u, 0u, 0u, 0u};
    const u32x4 a = (cvalid && e < p.q.dim) ? *(const u32x4*)(crow + (int64_t)e * 2) : (u32x4){0u, 0u, 0u, 0u};
    if (p.normalize & 1) ss += chunk_sumsq<EK>(b);
    acc = mfma32<EK>(acc, &a, &b);
  }
  ss += __shfl_xor(ss, 32);
  const float qsc = valid ? ((p.normalize & 1) ? inv_norm(ss) : 1.f) : 0.f;
  uint16_t* o = qc + q * qc_qs;
  const int slot = perm ? 16 * ((l32 >> 2) & 1) + 4 * (l32 >> 3) + (l32 & 3) : l32;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t row = tile * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
    if (row < p.pl.ncent) o[row * 32 + slot] = (uint16_t)f32_to_f16_bits(acc[i] * qsc);
  }
}

// tinv: inverse norms (ist = 4 bytes per token), or (code, inverse norm)
// records (ist = 8; the codes are still read from p.pl.codes), or null.
template <int EK, int DPAD, int NBITS, int QN, bool FULLD>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(QN > 1 ? 2 : 4)))
    plaid_qc_kernel(const Params p, const uint16_t* __restrict__ qc, int64_t qc_qs, const float* __restrict__ tinv,
                    int ist) {
  using T = KT<EK, DPAD>;
  constexpr int KS = T::KSTEPS;
  constexpr int HALF = DPAD / 2;
  constexpr int RSB = DPAD * NBITS / 8;            // residual bytes per (padded) row
  constexpr int NRI = (32 * RSB + 1023) / 1024;    // residual gather instructions per tile
  constexpr int RBL = HALF * NBITS / 8;            // residual bytes per lane
  constexpr int RVL = RBL / 4;
  constexpr int FPB = 8 / NBITS;
  constexpr int QCT = 32 * 64;                     // table rows of one query per tile
  constexpr int RES0 = QN * QCT;                   // stage offsets
  constexpr int INV0 = RES0 + NRI * 1024;
  constexpr int STB = INV0 + 256;  // norms: 32 floats, or 32 records' (4-byte shifted)
  // vector memory instructions issued per iteration: the gather (table rows,
  // residual bytes, norms: G) and one code load, all loads into LDS, which
  // return in issue order, so a fixed count identifies the tile in flight
  constexpr int G = 2 * QN + NRI + 1;
  static_assert(RBL % 4 == 0, "residual lane bytes");
  static_assert(G + 1 <= 63, "vmcnt range");
  constexpr float NEG_INF = -__builtin_huge_valf();

  // byte -> its fields' bucket weights rounded to the MFMA type, packed in pairs
  __shared__ __attribute__((aligned(16))) float s_lut[2 * 256];
  // two stages per wave: tile c is read from one while tile c+1 lands in the other
  __shared__ __attribute__((aligned(1024))) char s_st[4][2][STB];
  // codes of tiles c+2 .. c+4 (slot t % 4), loaded two iterations ahead of their gather
  __shared__ __attribute__((aligned(16))) int32_t s_codes[4][4][32];
  // this wave's doc scores, written to memory once after its loop
  __shared__ float s_out[4][QN][kQcRMax];
  // this wave's doc boundaries (cu_seqlens[j0 .. j1]), read from LDS in the
  // loop at doc ends only: a vector load there would make the compiler wait
  // for every load in flight, the gathers included
  __shared__ int32_t s_cu[4][kQcRMax + 1];
  for (int v = threadIdx.x; v < 256; v += 256) {
    uint32_t h16[4] = {0u, 0u, 0u, 0u};
    for (int k = 0; k < FPB; ++k) {
      uint32_t bc = ((uint32_t)v >> (k * NBITS)) & ((1u << NBITS) - 1u);
      bc = bc < (uint32_t)p.pl.nb ? bc : (uint32_t)(p.pl.nb - 1);
      const float wgt = p.pl.bw[bc];
      h16[k] = EK == EK_F16 ? f32_to_f16_bits(wgt) : f32_to_bf16_bits(wgt);
    }
    uint32_t* e = (uint32_t*)&s_lut[v * 2];
    e[0] = h16[0] | (h16[1] << 16);
    e[1] = h16[2] | (h16[3] << 16);
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
  const int wl = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t wv = (int64_t)blockIdx.x * 4 + wl;
  const int64_t g = wv / p.NR, r = wv - g * p.NR;
  if (g >= p.ngroups) return;  // wave-uniform, after the only barrier

  // ---- queries g * QN + sub: token l32 of each in column l32 ----
  u32x4 bq[QN][KS];
  float qsc[QN];
  const bool f_norm_q = (p.normalize & 1) != 0;
#pragma unroll
  for (int sub = 0; sub < QN; ++sub) {
    const int64_t q = g * QN + sub;
    const bool valid = q < p.q.n && l32 < seq_len(p.q, q);
    const char* rowp = valid ? seq_row0(p.q, q) + (int64_t)l32 * p.q.sl_b : nullptr;
    float ss = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int e = h * HALF + ks * 8;
      bq[sub][ks] = (valid && (FULLD || e < p.q.dim)) ? *(const u32x4*)(rowp + (int64_t)e * 2)
                                                      : (u32x4){0u, 0u, 0u, 0u};
      if (f_norm_q) ss += chunk_sumsq<EK>(bq[sub][ks]);
    }
    ss += __shfl_xor(ss, 32);
    qsc[sub] = valid ? (f_norm_q ? inv_norm(ss) : 1.f) : 0.f;
    // complete the fragment loads here: a load still pending in the
    // compiler's view at the loop would put a full vmcnt(0) wait (all the
    // gathers in flight) in front of every tile's MFMAs
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(bq[sub][ks]));
  }

  // ---- this wave's docs [j0, j1): tokens [T0, T1) of the packed corpus ----
  const int64_t j0 = r * p.R;
  const int64_t j1 = j0 + p.R < p.pl.n ? j0 + p.R : p.pl.n;
  const int nd = (int)(j1 - j0);
  for (int k = lane; k <= nd; k += 64) s_cu[wl][k] = p.pl.cu[j0 + k];
  __builtin_amdgcn_wave_barrier();
  // tokens are counted from T0 (the range spans < 2^31 tokens)
  const int T0 = __builtin_amdgcn_readfirstlane(s_cu[wl][0]);
  const int span = __builtin_amdgcn_readfirstlane(s_cu[wl][nd]) - T0;
  const int ntile = (span + 31) >> 5;

  // raw buffer descriptor words (stride 0, untyped 32-bit format)
  auto rsrc_words = [](const void* base, uint32_t nbytes) -> u32x4 {
    const uint64_t b = (uint64_t)base;
    return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b),
                 (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32) & 0xffffu),
                 (uint32_t)__builtin_amdgcn_readfirstlane(nbytes), 0x00020000u};
  };
  // the queries' tables (a query past the batch reads zeros: record count 0);
  // rows past the tile's end get offset kInvRow, beyond every table
  u32x4 dqc[QN];
#pragma unroll
  for (int sub = 0; sub < QN; ++sub) {
    const int64_t q = g * QN + sub;
    dqc[sub] = rsrc_words(qc + (q < p.q.n ? q : 0) * qc_qs, q < p.q.n ? (uint32_t)(p.pl.ncent * 64) : 0u);
  }
  // LDS addresses of the two stages and of code slot 0 (loop constants)
  uint32_t st_lds[2];
#pragma unroll
  for (int k = 0; k < 2; ++k)
    st_lds[k] = (uint32_t)__builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)(&s_st[wl][k][0]));
  const uint32_t cs_lds0 = (uint32_t)__builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int32_t*)(&s_codes[wl][0][0]));
  // (s_nop 4: the descriptor words come from v_readlane / v_readfirstlane,
  // VALU writes of SGPRs that a VMEM instruction may read only 5 wait states
  // later; the compiler does not count wait states into inline asm)
  auto dma = [&](uint32_t lds, uint32_t voff, const u32x4& desc) {
    uint32_t saved;
    asm volatile(
        "s_nop 4\n\t"
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"  // an M0 write needs one wait state before an LDS DMA reads it
        "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(lds), "v"(voff), "s"(desc)
        : "memory");
  };
  auto dma_nt = [&](uint32_t lds, uint32_t voff, const u32x4& desc) {
    uint32_t saved;
    asm volatile(
        "s_nop 4\n\t"
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"  // an M0 write needs one wait state before an LDS DMA reads it
        "buffer_load_dwordx4 %2, %3, 0 offen nt lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(lds), "v"(voff), "s"(desc)
        : "memory");
  };
  // Table rows land at row positions P(R) = R ^ ((R >> 2) & 1): the rows
  // R and R + 4 that one fragment read touches (lanes of the two halves)
  // then sit in different banks. Instruction i fills positions 16 i + lane / 4.
  auto rowpos = [](int row) { return row ^ ((row >> 2) & 1); };
  // Tiles are 32 consecutive tokens of the range, tile i at T0 + 32 i, in
  // whichever docs they fall; a tile past the range loads nothing (record
  // count 0). The streams' base addresses advance by one tile per iteration
  // (64-bit scalar adds; no multiplies in the loop).
  auto rows_of = [&](int i) {  // rows of tile i that exist
    const int rem = span - 32 * i;
    return rem < 0 ? 0 : (rem < 32 ? rem : 32);
  };
  const char* code_p = (const char*)(p.pl.codes + T0);  // tile 0
  const char* res_p = (const char*)p.pl.res + (int64_t)T0 * p.pl.res_st;
  // a record's norm is its second word: the norms' stream starts 4 bytes in
  const char* inv_p = tinv ? (const char*)tinv + (int64_t)T0 * ist + (ist == 8 ? 4 : 0) : nullptr;
  const int inv_tile = 32 * ist;
  const int64_t res_tile = 32 * p.pl.res_st;
  // codes of tile i (at code_p) into code slot `slot` (lanes 0..7, 16 bytes each)
  auto code_dma = [&](int i, int slot, const char* cp) {
    const u32x4 dc = rsrc_words(cp, (uint32_t)rows_of(i) * 4u);
    if (lane < 8) dma_nt(cs_lds0 + (uint32_t)(slot * 128), (uint32_t)(lane * 16), dc);
  };
  // gather tile i (code of row l32 in code slot `slot`) into stage `stage`,
  // once the stage's previous contents have been read (lgkmcnt(0)); exactly
  // G load instructions whether or not the tile exists
  auto gather = [&](int i, int slot, int stage, const char* rp, const char* ip) {
    const int nv = rows_of(i);
    const uint32_t cd = (uint32_t)s_codes[wl][slot][l32];
    const uint32_t rowoff = l32 < nv ? (cd < (uint32_t)p.pl.ncent ? cd : 0u) * 64u : kInvRow;
    uint32_t voff[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int row = rowpos(k * 16 + lane / 4);  // P is its own inverse
      voff[k] = (uint32_t)__builtin_amdgcn_ds_bpermute(row * 4, (int)rowoff) + (uint32_t)((lane & 3) * 16);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int sub = 0; sub < QN; ++sub)
#pragma unroll
      for (int k = 0; k < 2; ++k) dma(st_lds[stage] + (uint32_t)(sub * QCT + k * 1024), voff[k], dqc[sub]);
    const u32x4 dres = rsrc_words(rp, (uint32_t)nv * (uint32_t)p.pl.res_st);
#pragma unroll
    for (int k = 0; k < NRI; ++k) dma_nt(st_lds[stage] + (uint32_t)(RES0 + k * 1024), (uint32_t)(k * 1024 + lane * 16), dres);
    // norms (records: every other word, from 4 bytes in, so the byte count
    // stops at the last row's norm and nothing past the array is read)
    const uint32_t inb = nv == 0 ? 0u : (uint32_t)(nv * ist - (ist == 8 ? 4 : 0));
    const u32x4 dinv = rsrc_words(ip ? (const void*)ip : (const void*)p.pl.res, ip ? inb : 0u);
    if (lane < 2 * ist) dma_nt(st_lds[stage] + (uint32_t)INV0, (uint32_t)(lane * 16), dinv);
  };

  float m[QN];
  int rot0[QN];  // first 4-column chunk of each query's flush order (loop-invariant)
#pragma unroll
  for (int sub = 0; sub < QN; ++sub) {
    m[sub] = NEG_INF;
    rot0[sub] = (p.LU & 3) == 0 ? (int)((g * QN + sub) % (p.LU >> 2)) : 0;
  }

  struct Regs {
    uint32_t rw[RVL];
    f32x4 inv[4];
    f16x2 qv[QN][8];  // table values of the lane's 16 rows, two per register
  };
  // lane-constant LDS offsets within a stage: residual bytes of row l32's
  // half h; table row positions P(row) = 8a + 4h + (b ^ h) for row
  // 8a + 4h + b, i.e. + h for even b and - h for odd b
  const int res_lane = RES0 + l32 * (int)p.pl.res_st + h * RBL;
  const int qv_even = (4 * h + h) * 64 + l32 * 2, qv_odd = (4 * h - h) * 64 + l32 * 2;
  auto read_stage = [&](Regs& rg, int stage, auto NORMD) {
    const char* st = &s_st[wl][stage][0];
    const char* rp = st + res_lane;
    if constexpr (RVL % 4 == 0) {
#pragma unroll
      for (int v = 0; v < RVL / 4; ++v) {
        const u32x4 t = *(const u32x4*)(rp + 16 * v);
        rg.rw[4 * v] = t[0]; rg.rw[4 * v + 1] = t[1]; rg.rw[4 * v + 2] = t[2]; rg.rw[4 * v + 3] = t[3];
      }
    } else {
#pragma unroll
      for (int v = 0; v < RVL / 2; ++v) {
        const uint2 t = *(const uint2*)(rp + 8 * v);
        rg.rw[2 * v] = t.x; rg.rw[2 * v + 1] = t.y;
      }
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      constexpr int NM = decltype(NORMD)::value;  // 0: none, 1: norms, 2: records
      if constexpr (NM == 2) {
        const f32x4 a = *(const f32x4*)(st + INV0 + (8 * jj + 4 * h) * 8);
        const f32x4 b = *(const f32x4*)(st + INV0 + (8 * jj + 4 * h) * 8 + 16);
        rg.inv[jj] = (f32x4){a[0], a[2], b[0], b[2]};
      } else {
        rg.inv[jj] = NM ? *(const f32x4*)(st + INV0 + (8 * jj + 4 * h) * 4) : (f32x4){1.f, 1.f, 1.f, 1.f};
      }
    }
#pragma unroll
    for (int sub = 0; sub < QN; ++sub)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int rel = (8 * (i >> 2) + (i & 3)) * 64 + sub * QCT;  // compile-time
        rg.qv[sub][i >> 1][i & 1] = *(const _Float16*)(st + ((i & 1) ? qv_odd : qv_even) + rel);
      }
  };
  // a * b + (fp16 half of w), one v_fma_mix_f32 (the half converted
  // exactly). Written as fmaf on the converted half, not as inline asm: the
  // operand a comes straight from an MFMA, and only for compiler-visible
  // instructions does the compiler insert the wait states an MFMA result
  // needs before a VALU instruction may read it.
  auto fma_mix = [](float a, float b, f16x2 w, auto HI) -> float {
    return __builtin_fmaf(a, b, (float)w[decltype(HI)::value ? 1 : 0]);
  };
  // The doc whose tokens continue into the current tile (jc, ending at token
  // ec); its end is known without a table read until it is reached.
  int jc = 0;
  int ec = __builtin_amdgcn_readfirstlane(s_cu[wl][1]) - T0;  // relative to T0
  // park doc jc's maxima (sum over the query's columns in the tile kernel's
  // order) and move to the next doc
  auto doc_end = [&]() {
#pragma unroll
    for (int sub = 0; sub < QN; ++sub) {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(m[sub]), __float_as_uint(m[sub]), false, false);
      const float mm = max_nan(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
      const float v = __builtin_isfinite(mm) ? mm : 0.f;
      auto col = [&](int c) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), c)); };
      // the tile kernel's flush order (query g at place g of its group of 4:
      // the sum starts at 4-column chunk g % (Lq / 4) and wraps)
      float sum = 0.f;
      if ((p.LU & 3) == 0) {
        const int nv4 = p.LU >> 2;
        int c = rot0[sub];
        for (int jj = 0; jj < nv4; ++jj) {
          sum += col(4 * c);
          sum += col(4 * c + 1);
          sum += col(4 * c + 2);
          sum += col(4 * c + 3);
          c = (c + 1 == nv4) ? 0 : c + 1;
        }
      } else {
        for (int c = 0; c < p.LU; ++c) sum += col(c);
      }
      if (lane == 0) s_out[wl][sub][jc] = sum * p.out_scale;
      m[sub] = NEG_INF;
    }
    ++jc;
    ec = jc < nd ? __builtin_amdgcn_readfirstlane(s_cu[wl][jc + 1]) - T0 : 0x7fffffff;
  };
  auto compute = [&](int i, const Regs& rg) {
    const int T = 32 * i;  // relative to T0
    f32x16 acc[QN];
    const uint32_t* rw = rg.rw;
    auto byte_at = [&](int byte_i) -> uint32_t { return (rw[byte_i >> 2] >> ((byte_i & 3) * 8)) & 0xffu; };
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 rv;
      if constexpr (FPB == 4) {
        const uint2 e0 = *(const uint2*)&s_lut[byte_at(2 * ks) * 2];
        const uint2 e1 = *(const uint2*)&s_lut[byte_at(2 * ks + 1) * 2];
        rv = u32x4{e0.x, e0.y, e1.x, e1.y};
      } else if constexpr (FPB == 2) {
#pragma unroll
        for (int k = 0; k < 4; ++k) rv[k] = *(const uint32_t*)&s_lut[byte_at(4 * ks + k) * 2];
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t b0 = byte_at(8 * ks + 2 * k), b1 = byte_at(8 * ks + 2 * k + 1);
          rv[k] = (*(const uint32_t*)&s_lut[b0 * 2] & 0xffffu) | (*(const uint32_t*)&s_lut[b1 * 2] << 16);
        }
      }
      u32x4 ra = rv;
      if constexpr (!FULLD) {
        if ((h * HALF + ks * 8) >= p.q.dim) ra = (u32x4){0u, 0u, 0u, 0u};  // chunks are whole: dim % 8 == 0
      }
#pragma unroll
      for (int sub = 0; sub < QN; ++sub) acc[sub] = mfma32<EK>(ks == 0 ? f32x16{} : acc[sub], &ra, &bq[sub][ks]);
    }
    if (ec - T > 32) {
      // the whole tile belongs to doc jc (the common case)
#pragma unroll
      for (int sub = 0; sub < QN; ++sub)
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
          const float v0 = fma_mix(acc[sub][e], qsc[sub], rg.qv[sub][e >> 1], std::false_type{}) * rg.inv[e >> 2][e & 3];
          const float v1 = fma_mix(acc[sub][e + 1], qsc[sub], rg.qv[sub][e >> 1], std::true_type{}) *
                           rg.inv[(e + 1) >> 2][(e + 1) & 3];
          m[sub] = max_nan(m[sub], max_nan(v0, v1));
        }
      return;
    }
    // doc ends inside the tile: rows [a, b) of each doc in turn (values
    // recomputed per segment: holding them would cost 16 registers a query)
    int a = 0;
    while (true) {
      const int b = ec - T < 32 ? ec - T : 32;
      const int la = a - 4 * h, lb = b - 4 * h;  // row r = 8 (e / 4) + 4 h + e % 4
#pragma unroll
      for (int sub = 0; sub < QN; ++sub)
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
          const float v0 = fma_mix(acc[sub][e], qsc[sub], rg.qv[sub][e >> 1], std::false_type{}) * rg.inv[e >> 2][e & 3];
          const float v1 = fma_mix(acc[sub][e + 1], qsc[sub], rg.qv[sub][e >> 1], std::true_type{}) *
                           rg.inv[(e + 1) >> 2][(e + 1) & 3];
          const int r0 = 8 * (e >> 2) + (e & 3);
          m[sub] = max_nan(m[sub], max_nan((r0 >= la && r0 < lb) ? v0 : NEG_INF, (r0 + 1 >= la && r0 + 1 < lb) ? v1 : NEG_INF));
        }
      if (ec - T > 32 || jc >= nd) break;  // doc jc continues in the next tile
      doc_end();
      a = b;
    }
  };

  // Pipeline: at the top of iteration c, tile c's gather (stage c % 2) and
  // the codes of tile c + 2 (slot (c + 2) % 4) have landed; tile c + 1's
  // gather and the codes of tile c + 3 may be in flight (G + 1 loads).
  // Iteration c reads its stage, gathers tile c + 2 into it, loads the codes
  // of tile c + 4, then scores tile c.
  code_dma(0, 0, code_p);
  code_dma(1, 1, code_p + 128);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  gather(0, 0, 0, res_p, inv_p);
  code_dma(2, 2, code_p + 256);
  gather(1, 1, 1, res_p + res_tile, inv_p ? inv_p + inv_tile : nullptr);
  code_dma(3, 3, code_p + 384);
  // (two copies of the loop: with and without token inverse norms)
  auto scan = [&](auto NORMD) {
    const char* cp = code_p + 512;                 // tile c + 4
    const char* rp = res_p + 2 * res_tile;         // tile c + 2
    const char* ip = NORMD ? inv_p + 2 * inv_tile : nullptr;
    for (int c = 0; c < ntile; ++c) {
      asm volatile("s_waitcnt vmcnt(%0)" : : "n"(G + 1) : "memory");
      const int stage = c & 1;
      Regs rg;
      read_stage(rg, stage, NORMD);
      gather(c + 2, (c + 2) & 3, stage, rp, ip);
      code_dma(c + 4, c & 3, cp);
      compute(c, rg);
      cp += 128;
      rp += res_tile;
      if (NORMD) ip += inv_tile;
    }
  };
  if (tinv && ist == 8)
    scan(std::integral_constant<int, 2>{});
  else if (tinv)
    scan(std::integral_constant<int, 1>{});
  else
    scan(std::integral_constant<int, 0>{});
  // docs left (empty docs at the range's end, or an empty range)
  while (jc < nd) doc_end();
  // no gather may still be writing this wave's LDS when it exits
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // this wave's doc scores (written by lane 0: visible to the whole wave)
  __builtin_amdgcn_wave_barrier();
  for (int k = lane; k < nd; k += 64)
#pragma unroll
    for (int sub = 0; sub < QN; ++sub) {
      const int64_t q = g * QN + sub;
      if (q < p.q.n) p.out[q * p.osq + (j0 + k) * p.osd] = s_out[wl][sub][k];
    }
}

// ---------------------------------------------------------------------------
// plaid_scan_kernel: the same scan with query tokens as the MFMA A rows and
// doc tokens as the B columns, one doc token per lane (l32), so that every
// stream lands in registers with plain buffer loads and no LDS staging:
//   lane (l32, h) of tile t loads token l32's code, its residual bytes of
//   half h (16 B at d = 128, nbits = 2), its inverse norm, and 32 bytes of
//   table rows: the table stores the 16 query slots of half h contiguously
//   (query token s at slot 16 ((s >> 2) & 1) + 4 (s >> 3) + (s & 3), the
//   accumulator order of element e of that half), and the lane reads 16 of
//   them from each of the rows of tokens l32 % 16 and l32 % 16 + 16, so that
//   the four lanes reading one row in a load sit in one 64-byte request;
//   v_permlane16_swap then hands each lane its own token's 32 bytes.
// The accumulator element e of lane (l32, h) is query token
// 8 (e / 4) + 4 h + e % 4 against doc token l32; the query rows are
// normalised before they are rounded, so the epilogue is
//   v[e] = (acc[e] + qc[e]) * inv      (inv: one value per lane)
// and the running max is elementwise per lane across tiles; a doc's end
// reduces the 16 maxima of each half over its 32 lanes (a transposing
// butterfly of permlane16 swaps and DPP moves) and sums the 32 query tokens.
// Pipeline: tile c + LS's loads are issued after tile c is scored; their
// codes were loaded LC = 2 LS tiles ahead, right after tile c's loads, so a
// wait for either never waits for a younger load. With token records (REC)
// the code and the norm of a token come in one record, and the records of
// two tiles in one 64-lane load every other step (see the REC branch at the
// loop). The loads are inline asm with explicit vmcnt counts (see
// load_tile). The loop is unrolled by LC so the register rings have static
// indices.
// Measured on the C5 corpus at Nq = 1: 2.70 ms with the LDS-staged kernel;
// 2.57 ms register-direct; 2.40 ms with table reads of 16 rows per load
// (four lanes per row, above) instead of 32 rows by two lanes each; 2.32 ms
// with records; 2.245 ms with records of two tiles per load. What bounds it
// (counters): the texture data unit, busy 0.955 of the cycles returning 832
// dwords per tile to registers (512 of them table rows). Tried: the streamed
// bytes through an 8-tile LDS ring (buffer_load ... lds, 2.6x the bytes in
// flight, 128 VGPRs): 2.60 against 2.57 ms, and the same at four waves per
// SIMD with 6 tiles: 2.75 ms; so latency is not the bound.
// Steps I .. N-1 of one unrolled round (static register indices), stopping
// at the last tile; false once it stopped.
template <int I, int N, class F>
__device__ __forceinline__ bool scan_steps(F& f, int c, int n) {
  if constexpr (I == N) {
    return true;
  } else {
    if (c + I >= n) return false;
    f(std::integral_constant<int, I>{}, c + I);
    return scan_steps<I + 1, N>(f, c, n);
  }
}

// LS tiles in flight per wavefront: 3 at three waves per SIMD, 2 at four.
// REC: tinv points at (code, inverse norm) records of 8 bytes per token
// (lik_plaid_token_t), read in place of the codes and the norms by one load.
// QN: queries per wavefront (2 with records: both score the same residual
// bytes and records, each from its own table; two waves per SIMD).
template <int EK, int DPAD, int NBITS, bool FULLD, bool NORMD, int LS, bool REC, int QN = 1>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(QN == 2 ? 2 : (LS == 2 ? 4 : 3))))
    plaid_scan_kernel(const Params p, const uint16_t* __restrict__ qc, int64_t qc_qs, const float* __restrict__ tinv) {
  using T = KT<EK, DPAD>;
  constexpr int KS = T::KSTEPS;
  constexpr int HALF = DPAD / 2;
  constexpr int RBL = HALF * NBITS / 8;  // residual bytes per lane (8 .. 64)
  constexpr int RW = RBL / 4;            // ... as dwords
  constexpr int FPB = 8 / NBITS;
  constexpr int LC = 2 * LS;
  constexpr uint32_t NT = 2;  // non-temporal cache policy of the streamed loads
  constexpr float NEG_INF = -__builtin_huge_valf();
  static_assert(RW == 2 || RW % 4 == 0, "residual lane bytes");
  static_assert(QN == 1 || (QN == 2 && REC), "two queries per wavefront with records only");

  __shared__ __attribute__((aligned(16))) float s_lut[2 * 256];
  __shared__ float s_out[4][QN][kQcRMax];
  __shared__ int32_t s_cu[4][kQcRMax + 1];
  for (int v = threadIdx.x; v < 256; v += 256) {
    uint32_t h16[4] = {0u, 0u, 0u, 0u};
    for (int k = 0; k < FPB; ++k) {
      uint32_t bc = ((uint32_t)v >> (k * NBITS)) & ((1u << NBITS) - 1u);
      bc = bc < (uint32_t)p.pl.nb ? bc : (uint32_t)(p.pl.nb - 1);
      const float wgt = p.pl.bw[bc];
      h16[k] = EK == EK_F16 ? f32_to_f16_bits(wgt) : f32_to_bf16_bits(wgt);
    }
    uint32_t* e = (uint32_t*)&s_lut[v * 2];
    e[0] = h16[0] | (h16[1] << 16);
    e[1] = h16[2] | (h16[3] << 16);
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
  const int wl = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t wv = (int64_t)blockIdx.x * 4 + wl;
  const int64_t g = wv / p.NR, r = wv - g * p.NR;
  if (g >= p.ngroups) return;  // wave-uniform, after the only barrier

  // ---- queries g QN + sub: token l32 as the A rows (the B columns of the
  // other kernels), scaled by its inverse norm before rounding (0 past its
  // length), so the accumulators are q^.r and the table holds q^.c ----
  u32x4 aq[QN][KS];
#pragma unroll
  for (int sub = 0; sub < QN; ++sub) {
    const int64_t q = g * QN + sub;
    const bool valid = q < p.q.n && l32 < seq_len(p.q, q);
    const char* rowp = valid ? seq_row0(p.q, q) + (int64_t)l32 * p.q.sl_b : nullptr;
    float ss = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int e = h * HALF + ks * 8;
      aq[sub][ks] = (valid && (FULLD || e < p.q.dim)) ? *(const u32x4*)(rowp + (int64_t)e * 2) : (u32x4){0u, 0u, 0u, 0u};
      if (p.normalize & 1) ss += chunk_sumsq<EK>(aq[sub][ks]);
    }
    ss += __shfl_xor(ss, 32);
    const float sc = valid ? ((p.normalize & 1) ? inv_norm(ss) : 1.f) : 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t x = aq[sub][ks][w];
        if constexpr (EK == EK_F16)
          aq[sub][ks][w] = f32_to_f16_bits(f16_to_f32((uint16_t)(x & 0xffffu)) * sc) |
                           (f32_to_f16_bits(f16_to_f32((uint16_t)(x >> 16)) * sc) << 16);
        else
          aq[sub][ks][w] = f32_to_bf16_bits(bf16lo_to_f32(x) * sc) | (f32_to_bf16_bits(bf16hi_to_f32(x) * sc) << 16);
      }
      asm volatile("" : "+v"(aq[sub][ks]));
    }
  }

  // ---- this wave's docs [j0, j1): tokens [T0, T0 + span) of the packed corpus ----
  const int64_t j0 = r * p.R;
  const int64_t j1 = j0 + p.R < p.pl.n ? j0 + p.R : p.pl.n;
  const int nd = (int)(j1 - j0);
  for (int k = lane; k <= nd; k += 64) s_cu[wl][k] = p.pl.cu[j0 + k];
  __builtin_amdgcn_wave_barrier();
  const int T0 = __builtin_amdgcn_readfirstlane(s_cu[wl][0]);
  const int span = __builtin_amdgcn_readfirstlane(s_cu[wl][nd]) - T0;
  const int ntile = (span + 31) >> 5;

  // codes (4 bytes per token), or records (8 bytes: code, inverse norm)
  const char* code_p = REC ? (const char*)(tinv + 2 * (int64_t)T0) : (const char*)(p.pl.codes + T0);
  const char* res_p = (const char*)p.pl.res + (int64_t)T0 * p.pl.res_st;
  const float* inv_p = (NORMD && !REC) ? tinv + T0 : nullptr;
  const int64_t res_tile = 32 * p.pl.res_st;
  const uint32_t res_lane = (uint32_t)(l32 * p.pl.res_st + h * RBL);
  auto rows_of = [&](int i) {
    const int rem = span - 32 * i;
    return rem < 0 ? 0 : (rem < 32 ? rem : 32);
  };
  // Loads are inline asm into registers, waited for by explicit vmcnt
  // counts (loads return in issue order): with compiler-visible loads the
  // compiler's own wait insertion puts a full vmcnt(0) at the loop head.
  // A load's destination registers are tied to the stage's previous
  // contents ("+v"), so each ring slot keeps its physical registers from
  // one load to the next and the register allocator never moves (reads) a
  // register whose load is still in flight; each wait names the registers it
  // guards, so nothing reads a stage before its wait; and the loads of a step
  // are issued after an ordering point on the running maxima, which every
  // read of the previous contents feeds. Descriptors: raw, stride 0, untyped.
  // Each load starts with s_nop 4: its descriptor words come from
  // v_readfirstlane (a VALU write of SGPRs), which a VMEM instruction may read
  // only 5 wait states later, and the compiler does not count wait states
  // into inline asm.
  auto desc = [](const void* base, uint32_t nbytes) -> u32x4 {
    const uint64_t b = (uint64_t)base;
    return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b),
                 (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32) & 0xffffu),
                 (uint32_t)__builtin_amdgcn_readfirstlane(nbytes), 0x00020000u};
  };
  // the queries' tables (a query past the batch reads zeros: record count 0)
  u32x4 dtab[QN];
#pragma unroll
  for (int sub = 0; sub < QN; ++sub) {
    const int64_t q = g * QN + sub;
    dtab[sub] = desc(qc + (q < p.q.n ? q : 0) * qc_qs, q < p.q.n ? (uint32_t)(p.pl.ncent * 64) : 0u);
  }

  struct Stage {
    u32x4 rw[RW == 2 ? 1 : RW / 4];  // residual bytes (RW == 2: the low half of rw[0])
    float inv;
    u32x4 tq[QN][2];  // each table's 16 fp16 values of this lane's half, in element order
  };
  // loads per tile (residual, inverse norm, tables) and per code
  constexpr int NLT = (RW == 2 ? 1 : RW / 4) + ((NORMD && !REC) ? 1 : 0) + 2 * QN;
  Stage st[LS];
  uint32_t code[LC];  // (without records)
#pragma unroll
  for (int k = 0; k < LS; ++k) {
#pragma unroll
    for (int v = 0; v < (RW == 2 ? 1 : RW / 4); ++v) st[k].rw[v] = u32x4{0u, 0u, 0u, 0u};
    st[k].inv = 1.f;
#pragma unroll
    for (int sub = 0; sub < QN; ++sub) st[k].tq[sub][0] = st[k].tq[sub][1] = u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int k = 0; k < LC; ++k) code[k] = 0u;
  // codes and inverse norms: loaded by lanes 0..31 only (EXEC's high half
  // cleared inside the asm; the loop runs with all lanes active) and copied
  // to lanes 32..63 by v_permlane32_swap once they have arrived
  auto load_code = [&](int t, uint32_t& c) {
    const u32x4 dc = desc(code_p + 128 * (int64_t)t, (uint32_t)rows_of(t) * 4u);
    uint32_t ex;
    asm volatile("s_nop 4\n\ts_mov_b32 %1, exec_hi\n\ts_mov_b32 exec_hi, 0\n\t"
                 "buffer_load_dword %0, %2, %3, 0 offen nt\n\ts_mov_b32 exec_hi, %1"
                 : "+v"(c), "=&s"(ex) : "v"((uint32_t)l32 * 4u), "s"(dc));
  };
  auto bcast = [](uint32_t x) -> uint32_t {
    return __builtin_amdgcn_permlane32_swap(x, x, false, false)[0];
  };
  auto load_tile = [&](int t, uint32_t cd, Stage& s) {
    const int nv = rows_of(t);
    const u32x4 dr = desc(res_p + t * res_tile, (uint32_t)nv * (uint32_t)p.pl.res_st);
    if constexpr (RW == 2) {
      u32x2 v = {s.rw[0][0], s.rw[0][1]};
      asm volatile("s_nop 4\n\tbuffer_load_dwordx2 %0, %1, %2, 0 offen nt" : "+v"(v) : "v"(res_lane), "s"(dr));
      s.rw[0][0] = v[0];
      s.rw[0][1] = v[1];
    } else {
#pragma unroll
      for (int k = 0; k < RW / 4; ++k)
        asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2, 0 offen offset:%3 nt"
                     : "+v"(s.rw[k]) : "v"(res_lane), "s"(dr), "n"(16 * k));
    }
    if constexpr (NORMD && !REC) {
      const u32x4 di = desc(inv_p + 32 * (int64_t)t, (uint32_t)nv * 4u);
      uint32_t ex;
      asm volatile("s_nop 4\n\ts_mov_b32 %1, exec_hi\n\ts_mov_b32 exec_hi, 0\n\t"
                   "buffer_load_dword %0, %2, %3, 0 offen nt\n\ts_mov_b32 exec_hi, %1"
                   : "+v"(s.inv), "=&s"(ex) : "v"((uint32_t)l32 * 4u), "s"(di));
    }
    // table rows of tokens l32 % 16 (tq[0]) and l32 % 16 + 16 (tq[1]), 16
    // bytes each at quarter lane / 16 of the row, so four lanes read each row
    // of a load (16 rows per load instead of 32); unswap_table gives every
    // lane its own token's 32 bytes
    const auto cs = __builtin_amdgcn_permlane16_swap(cd, cd, false, false);
    const uint32_t qoff = (uint32_t)(lane >> 4) * 16u;
    const uint32_t ta = (cs[0] < (uint32_t)p.pl.ncent ? cs[0] : 0u) * 64u + qoff;
    const uint32_t tb = (cs[1] < (uint32_t)p.pl.ncent ? cs[1] : 0u) * 64u + qoff;
#pragma unroll
    for (int sub = 0; sub < QN; ++sub) {
      asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2, 0 offen" : "+v"(s.tq[sub][0]) : "v"(ta), "s"(dtab[sub]));
      asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2, 0 offen" : "+v"(s.tq[sub][1]) : "v"(tb), "s"(dtab[sub]));
    }
  };
  // Lane (l32, h) holds, of tokens l32 % 16 and l32 % 16 + 16, table quarter
  // 2 h + l32 / 16; one v_permlane16_swap per dword (odd rows of tq[0] with
  // even rows of tq[1]) leaves it quarters 2 h and 2 h + 1 of token l32: the
  // 16 values of its half, in element order.
  auto unswap_table = [](Stage& s) {
#pragma unroll
    for (int sub = 0; sub < QN; ++sub)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const auto sw = __builtin_amdgcn_permlane16_swap(s.tq[sub][0][k], s.tq[sub][1][k], false, false);
        s.tq[sub][0][k] = sw[0];
        s.tq[sub][1][k] = sw[1];
      }
  };
  // wait until at most n loads are in flight, for the registers of stage s
  auto wait_stage = [](auto NN, Stage& s) {
    constexpr int n = decltype(NN)::value;
    asm volatile("s_waitcnt vmcnt(%[n])" : "+v"(s.inv), "+v"(s.tq[0][0]), "+v"(s.tq[0][1]) : [n] "n"(n));
#pragma unroll
    for (int sub = 1; sub < QN; ++sub) asm volatile("" : "+v"(s.tq[sub][0]), "+v"(s.tq[sub][1]));
#pragma unroll
    for (int k = 0; k < (RW == 2 ? 1 : RW / 4); ++k) asm volatile("" : "+v"(s.rw[k]));
  };
  auto wait_code = [](auto NN, uint32_t& c) {
    asm volatile("s_waitcnt vmcnt(%1)" : "+v"(c) : "n"(decltype(NN)::value));
  };

  float m[QN][16];
#pragma unroll
  for (int sub = 0; sub < QN; ++sub)
#pragma unroll
    for (int e = 0; e < 16; ++e) m[sub][e] = NEG_INF;
  int jc = 0;
  int ec = __builtin_amdgcn_readfirstlane(s_cu[wl][1]) - T0;
  // doc jc ends: max over its lanes by a transposing butterfly (after the
  // step over lane bit b each lane keeps half of its values, so 16 values
  // take 8 + 4 + 2 + 1 + 1 exchanges): bit 4 by v_permlane16_swap, bits 3, 2,
  // 1, 0 by DPP (row_ror:8, row_half_mirror, quad_perm [3,2,1,0] and
  // [1,0,3,2]: each pairs lanes that differ in that bit); then the sum of the
  // 32 query tokens' maxima (non-finite -> 0) by a rotation all-reduce in a
  // fixed order. No LDS traffic.
  auto dpp = [](float x, auto CTRL) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), decltype(CTRL)::value, 0xf, 0xf, false));
  };
  using std::integral_constant;
  auto doc_end = [&]() {
#pragma unroll
   for (int sub = 0; sub < QN; ++sub) {
    float x[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // rows 0/1 and 2/3 swap: x[i] gets element i of lanes l, l^16 on even
      // rows and element i + 8 on odd rows
      const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(m[sub][i]), __float_as_uint(m[sub][i + 8]), false, false);
      x[i] = max_nan(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    }
    auto step = [&](int n, int bit, auto CTRL) {
#pragma unroll
      for (int i = 0; i < n; ++i) {
        const float keep = bit ? x[i + n] : x[i];
        const float send = bit ? x[i] : x[i + n];
        x[i] = max_nan(keep, dpp(send, CTRL));
      }
    };
    step(4, (l32 >> 3) & 1, integral_constant<int, 0x128>{});  // row_ror:8
    step(2, (l32 >> 2) & 1, integral_constant<int, 0x141>{});  // row_half_mirror
    step(1, (l32 >> 1) & 1, integral_constant<int, 0x1b>{});   // quad_perm [3,2,1,0]
    const float mm = max_nan(x[0], dpp(x[0], integral_constant<int, 0xb1>{}));  // quad_perm [1,0,3,2]
    float v = ((lane & 1) == 0 && __builtin_isfinite(mm)) ? mm : 0.f;
    v += dpp(v, integral_constant<int, 0x128>{});  // row_ror:8
    v += dpp(v, integral_constant<int, 0x124>{});  // row_ror:4
    v += dpp(v, integral_constant<int, 0x122>{});  // row_ror:2
    v += dpp(v, integral_constant<int, 0x121>{});  // row_ror:1
    {
      const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
      v = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
      v = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    if (lane == 0) s_out[wl][sub][jc] = v * p.out_scale;
#pragma unroll
    for (int e = 0; e < 16; ++e) m[sub][e] = NEG_INF;
   }
    ++jc;
    ec = jc < nd ? __builtin_amdgcn_readfirstlane(s_cu[wl][jc + 1]) - T0 : 0x7fffffff;
  };
  // a * one + (fp16 half of w): one v_fma_mix_f32 (compiler-visible, so the
  // MFMA-result wait states before it are the compiler's); `one` is an
  // opaque 1.0 so that the multiply is not folded into a convert + add
  float one = 1.f;
  asm volatile("" : "+s"(one));
  auto fma_mix = [&](float a, float, uint32_t w, auto HI) -> float {
    return __builtin_fmaf(a, one, (float)__builtin_bit_cast(f16x2, w)[decltype(HI)::value ? 1 : 0]);
  };
  auto compute = [&](int i, const Stage& s) {
    const int TT = 32 * i;
    f32x16 acc[QN];
    auto byte_at = [&](int byte_i) -> uint32_t {
      return (s.rw[byte_i >> 4][(byte_i >> 2) & 3] >> ((byte_i & 3) * 8)) & 0xffu;
    };
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 rv;
      if constexpr (FPB == 4) {
        const uint2 e0 = *(const uint2*)&s_lut[byte_at(2 * ks) * 2];
        const uint2 e1 = *(const uint2*)&s_lut[byte_at(2 * ks + 1) * 2];
        rv = u32x4{e0.x, e0.y, e1.x, e1.y};
      } else if constexpr (FPB == 2) {
#pragma unroll
        for (int k = 0; k < 4; ++k) rv[k] = *(const uint32_t*)&s_lut[byte_at(4 * ks + k) * 2];
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t b0 = byte_at(8 * ks + 2 * k), b1 = byte_at(8 * ks + 2 * k + 1);
          rv[k] = (*(const uint32_t*)&s_lut[b0 * 2] & 0xffffu) | (*(const uint32_t*)&s_lut[b1 * 2] << 16);
        }
      }
      if constexpr (!FULLD) {
        if ((h * HALF + ks * 8) >= p.q.dim) rv = (u32x4){0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int sub = 0; sub < QN; ++sub) acc[sub] = mfma32<EK>(ks == 0 ? f32x16{} : acc[sub], &aq[sub][ks], &rv);
    }
    // the tile's scores, in place of the accumulators
#pragma unroll
    for (int sub = 0; sub < QN; ++sub)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t w = s.tq[sub][e >> 3][(e >> 1) & 3];
        acc[sub][e] = ((e & 1) ? fma_mix(acc[sub][e], 1.f, w, std::true_type{})
                               : fma_mix(acc[sub][e], 1.f, w, std::false_type{})) * s.inv;
      }
    if (ec - TT > 32) {
#pragma unroll
      for (int sub = 0; sub < QN; ++sub)
#pragma unroll
        for (int e = 0; e < 16; ++e) m[sub][e] = max_nan(m[sub][e], acc[sub][e]);
      return;
    }
    int a = 0;
    while (true) {
      const int b = ec - TT < 32 ? ec - TT : 32;
      const bool in = l32 >= a && l32 < b;
#pragma unroll
      for (int sub = 0; sub < QN; ++sub)
#pragma unroll
        for (int e = 0; e < 16; ++e) m[sub][e] = max_nan(m[sub][e], in ? acc[sub][e] : NEG_INF);
      if (ec - TT > 32 || jc >= nd) break;
      doc_end();
      a = b;
    }
  };

  if constexpr (REC) {
    // Records two tiles at a time: one 64-lane load of tiles (u, u + 1), u
    // even (512 contiguous bytes; lanes 0..31 tile u, 32..63 tile u + 1),
    // into pair slot (u / 2) % 3. Odd step c issues the pair (c + 5, c + 6)
    // (into the slot of (c - 1, c), both scored by then) before tile c + 3's
    // loads. Loads issued after a tile's loads until its step: two steps of
    // NLT loads and one pair, 2 NLT + 1; after the pair holding tile c + 3's
    // record until step c issues that tile: 2 NLT + 1 at odd c, 3 NLT + 1 at
    // even c. The prologue issues what steps -5 .. -1 would have.
    static_assert(LS == 3 && LC == 6, "record pairs: three stages, a six-step round");
    u32x2 pr[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) pr[k] = u32x2{0u, 0u};
    auto load_pair = [&](int u, u32x2& v) {
      const u32x4 dc = desc(code_p + 256 * (int64_t)u, (uint32_t)(rows_of(u) + rows_of(u + 1)) * 8u);
      asm volatile("s_nop 4\n\tbuffer_load_dwordx2 %0, %1, %2, 0 offen nt" : "+v"(v) : "v"((uint32_t)lane * 8u), "s"(dc));
    };
    // word x of this lane's token in the even (lanes 0..31) or odd tile of a pair
    auto half = [](uint32_t x, auto ODD) -> uint32_t {
      const auto sw = __builtin_amdgcn_permlane32_swap(x, x, false, false);
      return decltype(ODD)::value ? sw[1] : sw[0];
    };
    using F = std::false_type;
    using Tt = std::true_type;
    load_pair(0, pr[0]);
    load_pair(2, pr[1]);
    asm volatile("s_waitcnt vmcnt(1)" : "+v"(pr[0]));
    load_tile(0, half(pr[0][0], F{}), st[0]);
    load_tile(1, half(pr[0][0], Tt{}), st[1]);
    load_pair(4, pr[2]);
    asm volatile("s_waitcnt vmcnt(%1)" : "+v"(pr[1]) : "n"(2 * NLT + 1));
    load_tile(2, half(pr[1][0], F{}), st[2]);
    auto step = [&](auto II, int c) {
      constexpr int I = decltype(II)::value;  // c % 6
      constexpr int J = (I + 3) % 6;           // (c + 3) % 6
      wait_stage(integral_constant<int, 2 * NLT + 1>{}, st[I % 3]);
      {
        Stage cur = st[I % 3];
        if constexpr (NORMD) cur.inv = __uint_as_float(half(pr[I / 2][1], integral_constant<bool, (I & 1) != 0>{}));
        unswap_table(cur);
        compute(c, cur);
      }
      // ordering point: the stage's previous contents are all read (they feed m)
#pragma unroll
      for (int e = 0; e < 16 * QN; ++e) asm volatile("" : "+v"(m[e / 16][e % 16]));
      if constexpr ((I & 1) != 0) load_pair(c + 5, pr[I / 2]);
      asm volatile("s_waitcnt vmcnt(%1)" : "+v"(pr[J / 2]) : "n"((I & 1) ? 2 * NLT + 1 : 3 * NLT + 1));
      load_tile(c + 3, half(pr[J / 2][0], integral_constant<bool, (J & 1) != 0>{}), st[I % 3]);
    };
    for (int c = 0; c < ntile; c += LC)
      if (!scan_steps<0, LC>(step, c, ntile)) break;
  } else {
    // Prologue: codes of tiles 0 .. LS-1; then for each t < LS tile t's loads
    // followed by the code of tile t + LS. From here on every tile's loads are
    // followed by exactly one code load, so at the top of step c tile c's loads
    // are followed by the code of tile c + LS and by LS - 1 later steps of
    // NLT + 1 loads each.
#pragma unroll
    for (int t = 0; t < LS; ++t) load_code(t, code[t]);
#pragma unroll
    for (int t = 0; t < LS; ++t) {
      asm volatile("s_waitcnt vmcnt(0)" : "+v"(code[t]));
      load_tile(t, bcast(code[t]), st[t]);
      load_code(t + LS, code[t + LS]);
    }
    constexpr int kWaitTile = 1 + (LS - 1) * (NLT + 1);
    auto step = [&](auto II, int c) {
      constexpr int I = decltype(II)::value;  // c % LC
      wait_stage(integral_constant<int, kWaitTile>{}, st[I % LS]);
      {
        Stage cur = st[I % LS];
        cur.inv = __uint_as_float(bcast(__float_as_uint(cur.inv)));
        unswap_table(cur);
        compute(c, cur);
      }
      // ordering point: the stage's previous contents are all read (they feed m)
#pragma unroll
      for (int e = 0; e < 16 * QN; ++e) asm volatile("" : "+v"(m[e / 16][e % 16]));
      // the code of tile c + LS, loaded right after tile c's loads
      wait_code(integral_constant<int, kWaitTile - 1>{}, code[(I + LS) % LC]);
      load_tile(c + LS, bcast(code[(I + LS) % LC]), st[I % LS]);
      load_code(c + LC, code[I]);
    };
    for (int c = 0; c < ntile; c += LC)
      if (!scan_steps<0, LC>(step, c, ntile)) break;
  }
  while (jc < nd) doc_end();
  // no load may still be writing this wave's registers when it exits
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __builtin_amdgcn_wave_barrier();
  for (int k = lane; k < nd; k += 64)
#pragma unroll
    for (int sub = 0; sub < QN; ++sub) {
      const int64_t q = g * QN + sub;
      if (q < p.q.n) p.out[q * p.osq + (j0 + k) * p.osd] = s_out[wl][sub][k];
    }
}

// out[q, j] = 0 for a query batch without tokens (Lq == 0)
__global__ void __launch_bounds__(256) zero_scores_kernel(float* out, int64_t nq, int64_t nd, int64_t osq,
                                                          int64_t osd) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < nq * nd) out[(i / nd) * osq + (i % nd) * osd] = 0.f;
}

template <int EK, int DPAD, int NBITS>
int launch_qc_scan(int qn, const Params& p, const uint16_t* qc, int64_t qc_qs, const float* tinv, bool rec, bool norm_d,
                   hipStream_t s) {
  const int64_t waves = p.ngroups * p.NR;
  const int64_t nb = (waves + 3) / 4;
  if (nb > 0x7fffffffLL) return LIK_ERR_UNSUPPORTED;
  const float* inv = norm_d ? tinv : nullptr;  // records are read for their norms only
  const int ist = rec ? 8 : 4;
  auto go = [&](auto kern) {
    launch_kernel(kern, dim3((unsigned)nb), dim3(256), 0, s, p, qc, qc_qs, inv, ist);
    return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
  };
  const bool full = p.q.dim == DPAD;
  if (qn == 2)
    return full ? go(plaid_qc_kernel<EK, DPAD, NBITS, 2, true>) : go(plaid_qc_kernel<EK, DPAD, NBITS, 2, false>);
  return full ? go(plaid_qc_kernel<EK, DPAD, NBITS, 1, true>) : go(plaid_qc_kernel<EK, DPAD, NBITS, 1, false>);
}

// Residual rows the register-direct scan takes: its loads land in registers
// that the compiler must neither spill nor copy while they are in flight, so
// only instantiations that compile without spills are built (2-bit rows, and
// 4-bit rows at d <= 64: 16 B of residual per lane); the others keep the
// LDS-staged scan.
constexpr int kScanLS = 3;  // (LS = 2 at four waves per SIMD spills at d = 128)

template <int DPAD, int NBITS>
constexpr bool scan_reg_ok() {
  return NBITS == 2 || (NBITS == 4 && DPAD == 64);
}

template <int EK, int DPAD, int NBITS>
int launch_scan(int qn, const Params& p, const uint16_t* qc, int64_t qc_qs, const float* tinv, bool rec, bool norm_d,
                hipStream_t s) {
  if constexpr (!scan_reg_ok<DPAD, NBITS>()) {
    return LIK_ERR_UNSUPPORTED;
  } else {
  const int64_t waves = p.ngroups * p.NR;
  const int64_t nb = (waves + 3) / 4;
  if (nb > 0x7fffffffLL) return LIK_ERR_UNSUPPORTED;
  auto go = [&](auto kern) {
    launch_kernel(kern, dim3((unsigned)nb), dim3(256), 0, s, p, qc, qc_qs, tinv);
    return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
  };
  const bool full = p.q.dim == DPAD;
  constexpr int LS = kScanLS;
  if (rec && qn == 2) {
    if (norm_d)
      return full ? go(plaid_scan_kernel<EK, DPAD, NBITS, true, true, LS, true, 2>)
                  : go(plaid_scan_kernel<EK, DPAD, NBITS, false, true, LS, true, 2>);
    return full ? go(plaid_scan_kernel<EK, DPAD, NBITS, true, false, LS, true, 2>)
                : go(plaid_scan_kernel<EK, DPAD, NBITS, false, false, LS, true, 2>);
  }
  if (qn != 1) return LIK_ERR_UNSUPPORTED;
  if (rec) {
    if (norm_d)
      return full ? go(plaid_scan_kernel<EK, DPAD, NBITS, true, true, LS, true>)
                  : go(plaid_scan_kernel<EK, DPAD, NBITS, false, true, LS, true>);
    return full ? go(plaid_scan_kernel<EK, DPAD, NBITS, true, false, LS, true>)
                : go(plaid_scan_kernel<EK, DPAD, NBITS, false, false, LS, true>);
  }
  if (norm_d)
    return full ? go(plaid_scan_kernel<EK, DPAD, NBITS, true, true, LS, false>)
                : go(plaid_scan_kernel<EK, DPAD, NBITS, false, true, LS, false>);
  return full ? go(plaid_scan_kernel<EK, DPAD, NBITS, true, false, LS, false>)
              : go(plaid_scan_kernel<EK, DPAD, NBITS, false, false, LS, false>);
  }
}

template <int EK, int DPAD>
int launch_qc(int qn, bool reg, const Params& p, uint16_t* qc, int64_t qc_qs, const float* tinv, bool rec,
              bool norm_d, hipStream_t s, const lik_launch_opts_t* opts) {
  const int64_t ntile = (p.pl.ncent + 31) / 32;
  const int64_t waves = p.q.n * ntile;
  if ((waves + 3) / 4 > 0x7fffffffLL) return LIK_ERR_UNSUPPORTED;
  // one query per wavefront: the register-direct scan, unless the caller
  // forces the LDS-staged one (plaid_variant 5)
  hipLaunchKernelGGL((centroid_scores_kernel<EK, DPAD>), dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, p, qc,
                     qc_qs, ntile, reg ? 1 : 0);
  if (hipGetLastError() != hipSuccess) return LIK_ERR_LAUNCH;
  TimingScope ts(opts);
  int rc;
  switch (p.pl.nbits) {
    case 2: rc = reg ? launch_scan<EK, DPAD, 2>(qn, p, qc, qc_qs, tinv, rec, norm_d, s)
                 : launch_qc_scan<EK, DPAD, 2>(qn, p, qc, qc_qs, tinv, rec, norm_d, s); break;
    case 4: rc = reg ? launch_scan<EK, DPAD, 4>(qn, p, qc, qc_qs, tinv, rec, norm_d, s)
                 : launch_qc_scan<EK, DPAD, 4>(qn, p, qc, qc_qs, tinv, rec, norm_d, s); break;
    case 8: rc = reg ? launch_scan<EK, DPAD, 8>(qn, p, qc, qc_qs, tinv, rec, norm_d, s)
                 : launch_qc_scan<EK, DPAD, 8>(qn, p, qc, qc_qs, tinv, rec, norm_d, s); break;
    default: rc = LIK_ERR_UNSUPPORTED;
  }
  const int rc2 = ts.close(s);
  return rc != LIK_OK ? rc : rc2;
}

}  // namespace lik

using namespace lik;

namespace {
constexpr int64_t kQcMaxQueries = 64;  // the table is per query: a few-query path

size_t qc_bytes(int64_t nq, int64_t ncent) { return (size_t)nq * (size_t)ncent * 64; }
}  // namespace

extern "C" size_t lik_plaid_maxsim_qc_workspace_size(const lik_seqs_t* Q, const lik_plaid_docs_t* docs) {
  if (!Q || !docs || Q->n < 0 || docs->n_centroids < 0) return 0;
  return (qc_bytes(Q->n, docs->n_centroids) + 255) & ~(size_t)255;
}

extern "C" int lik_plaid_maxsim_qc(const lik_seqs_t* Q, const lik_plaid_docs_t* docs, const float* token_inv,
                                   uint32_t flags, float* out, int64_t out_stride_q, int64_t out_stride_d,
                                   void* workspace, size_t workspace_bytes, const lik_launch_opts_t* opts,
                                   lik_stream_t stream) {
  if (!Q || !docs || Q->n < 0 || Q->len < 0 || docs->n < 0) return LIK_ERR_INVALID;
  if (Q->dtype != LIK_BF16 && Q->dtype != LIK_F16) return LIK_ERR_UNSUPPORTED;
  if (docs->centroid_dtype != Q->dtype) return LIK_ERR_UNSUPPORTED;
  if (docs->nbits != 2 && docs->nbits != 4 && docs->nbits != 8) return LIK_ERR_INVALID;
  if (docs->dim != Q->dim || Q->dim <= 0 || Q->dim % 8 != 0 || Q->dim > 128) return LIK_ERR_UNSUPPORTED;
  if (docs->n_buckets < 1 || docs->n_buckets > 256 || !docs->bucket_weights) return LIK_ERR_INVALID;
  if (!docs->cu_seqlens && !docs->lengths) return LIK_ERR_INVALID;
  if (!docs->cu_seqlens) return LIK_ERR_UNSUPPORTED;  // the scan walks the packed token stream
  if ((flags & LIK_KD_LAYOUT) || Q->mask || Q->token_scale || Q->cu_seqlens) return LIK_ERR_INVALID;
  if (Q->len > 32 || Q->n > kQcMaxQueries) return LIK_ERR_UNSUPPORTED;
  const bool norm_d = (flags & (LIK_NORMALIZE | LIK_NORMALIZE_D)) != 0;
  const bool rec = (flags & LIK_TOKEN_RECORDS) != 0;
  if ((norm_d || rec) && !token_inv) return LIK_ERR_INVALID;
  if (Q->n == 0 || docs->n == 0) return LIK_OK;
  if (!out) return LIK_ERR_INVALID;
  if (Q->len == 0) {
    // no query tokens: every score is 0 (the scan's column sums assume Lq > 0)
    const int64_t n = Q->n * docs->n;
    if ((n + 255) / 256 > 0x7fffffffLL) return LIK_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(zero_scores_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, out,
                       Q->n, docs->n, out_stride_q, out_stride_d);
    return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
  }
  if (!Q->data || !docs->codes || !docs->residuals || !docs->centroids || docs->n_centroids < 1)
    return LIK_ERR_INVALID;
  if (((uintptr_t)Q->data) % 16 || (Q->stride_l * 2) % 16 || (Q->stride_n * 2) % 16) return LIK_ERR_UNSUPPORTED;
  if (((uintptr_t)docs->centroids) % 16 != 0 || (docs->cent_stride * 2) % 16 != 0) return LIK_ERR_UNSUPPORTED;
  const int dpad = Q->dim <= 64 ? 64 : 128;
  const int64_t rsb = (int64_t)dpad * docs->nbits / 8, nri = (32 * rsb + 1023) / 1024;
  if (((uintptr_t)docs->residuals) % 16 != 0 || docs->res_stride_tok % 16 != 0 || 32 * docs->res_stride_tok > nri * 1024)
    return LIK_ERR_UNSUPPORTED;
  if (docs->res_stride_tok * 8 < (int64_t)docs->dim * docs->nbits) return LIK_ERR_INVALID;
  if (token_inv && ((uintptr_t)token_inv) % (rec ? 8 : 4)) return LIK_ERR_UNSUPPORTED;
  // table rows are gathered with 32-bit byte offsets below kInvRow
  if (docs->n_centroids * 64 >= (int64_t)kInvRow) return LIK_ERR_UNSUPPORTED;
  const size_t need = qc_bytes(Q->n, docs->n_centroids);
  if (!workspace || workspace_bytes < need || ((uintptr_t)workspace) % 16) return LIK_ERR_WORKSPACE;

  Params p{};
  p.q.data = (const char*)Q->data;
  p.q.sn_b = Q->stride_n * 2;
  p.q.sl_b = Q->stride_l * 2;
  p.q.lengths = Q->lengths;
  p.q.n = Q->n;
  p.q.L = Q->len;
  p.q.dim = Q->dim;
  p.pl.codes = docs->codes;
  p.pl.res = docs->residuals;
  p.pl.cu = docs->cu_seqlens;
  p.pl.lengths = docs->lengths;
  p.pl.n = docs->n;
  p.pl.L = docs->max_len;
  p.pl.codes_sn = docs->codes_stride_n;
  p.pl.res_st = docs->res_stride_tok;
  p.pl.cent = (const char*)docs->centroids;
  p.pl.cent_sb = docs->cent_stride * 2;
  p.pl.ncent = docs->n_centroids;
  p.pl.bw = docs->bucket_weights;
  p.pl.nb = docs->n_buckets;
  p.pl.nbits = docs->nbits;
  p.normalize = (flags & (LIK_NORMALIZE | LIK_NORMALIZE_Q)) ? 1 : 0;
  p.out_scale = 1.f;
  p.out = out;
  p.osq = out_stride_q;
  p.osd = out_stride_d;
  p.LU = (int)Q->len;
  // The register-direct scan wherever it applies (2-bit residuals, or 4-bit
  // at d <= 64): one query per wavefront from separate codes and norms
  // (faster per query than two queries per wavefront on the LDS-staged scan:
  // 2.25 against 2.56 ms at 8 queries, C5 corpus), two with token records
  // (they share each tile's residual bytes and records: 2.08 ms per query).
  // Otherwise the LDS-staged scan, two queries per wavefront when there are
  // several.
  const bool reg_ok = !(opts && opts->plaid_variant == 5) && (docs->nbits == 2 || (docs->nbits == 4 && dpad == 64));
  const int qn = Q->n < 2 ? 1 : reg_ok ? (rec ? 2 : 1) : 2;
  p.ngroups = (Q->n + qn - 1) / qn;
  // ~16k wavefronts over the corpus, at most kQcRMax docs each
  int64_t R = (docs->n + 16383) / 16384;
  if (opts && opts->docs_per_wg > 0) R = opts->docs_per_wg;
  p.R = (int)(R < 1 ? 1 : (R > kQcRMax ? kQcRMax : R));
  p.NR = (docs->n + p.R - 1) / p.R;
  uint16_t* qc = (uint16_t*)workspace;
  const int64_t qc_qs = docs->n_centroids * 32;
  // token_inv: inverse norms (used only when the docs are normalised), or
  // records (codes, and norms when normalised)
  const float* tinv = rec ? token_inv : norm_d ? token_inv : nullptr;
  hipStream_t s = (hipStream_t)stream;
  if (Q->dtype == LIK_BF16)
    return dpad == 64 ? launch_qc<EK_BF16, 64>(qn, reg_ok, p, qc, qc_qs, tinv, rec, norm_d, s, opts)
                      : launch_qc<EK_BF16, 128>(qn, reg_ok, p, qc, qc_qs, tinv, rec, norm_d, s, opts);
  return dpad == 64 ? launch_qc<EK_F16, 64>(qn, reg_ok, p, qc, qc_qs, tinv, rec, norm_d, s, opts)
                    : launch_qc<EK_F16, 128>(qn, reg_ok, p, qc, qc_qs, tinv, rec, norm_d, s, opts);
}
