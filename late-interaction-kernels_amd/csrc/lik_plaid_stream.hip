// PLAID residual MaxSim for a few queries (up to 4 of <= 32 tokens) on
// gfx950: one wavefront streams a range of documents for one query on its
// own, no LDS tile ring and no barriers in the loop.
//
// With a handful of query columns the tile kernel's per-tile work is mostly
// the decode and its latency chain (code -> centroid row -> decode -> MFMA);
// a workgroup walking thousands of tiles behind one barrier each is latency
// bound. Here each lane decodes the half row that is its own MFMA A fragment
// (lane (l32, h): doc token l32 of the tile, embedding elements
// [h*DPAD/2, (h+1)*DPAD/2)), the two halves' squared norms meet through one
// permlane32 swap, and the fragments go straight to the MFMA. Codes are
// loaded two tiles ahead and centroid rows / residual bytes one tile ahead
// (two staging sets), and several waves per SIMD cover the rest.
//
// The arithmetic is the decode kernel's (lik_plaid_decode.hip), element for
// element: emb = centroid + bucket weight in fp32, per 8-element chunk a fma
// chain of squares, chunk sums combined in the xor-tree order of a row's
// lanes, x / max(||x||, 1e-12) rounded once. The bucket weights of all fields
// of a residual byte come from one LDS table entry (byte -> values).
// Reference: plaid.py:684-963 (fused residual MaxSim), reference.py:124-179.
#include "lik_kernel.h"


namespace lik {

// Occupancy target: the latency chain is covered by the other waves of the
// SIMD, so registers are capped: 3 waves per SIMD at d <= 64, 2 at d = 128
// (query fragments, two staging sets of centroid rows and residual bytes,
// one accumulator; more waves would spill).
// FULLD: the embedding dim is DPAD (no padding elements to zero).
template <int EK, int DPAD, int CD, int NBITS, int NSUB, bool FULLD>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DPAD >= 128 ? 2 : 3)))
    plaid_stream_kernel(const Params p) {
  using T = KT<EK, DPAD>;
  constexpr int KS = T::KSTEPS;           // 8-element chunks per lane (= MFMA k-steps)
  constexpr int HALF = DPAD / 2;          // elements per lane
  constexpr int CSZ = CD == EK_F32 ? 4 : 2;
  constexpr int CVL = HALF * CSZ / 16;    // 16-byte centroid loads per lane
  constexpr int RBL = HALF * NBITS / 8;   // residual bytes per lane
  constexpr int RVL = RBL / 4;            // residual dwords per lane
  constexpr int FPB = 8 / NBITS;          // fields per residual byte
  static_assert(RBL % 4 == 0, "residual half rows are whole dwords");
  constexpr float NEG_INF = -__builtin_huge_valf();

  __shared__ __attribute__((aligned(16))) float s_lut[256 * FPB];
  for (int i = threadIdx.x; i < 256 * FPB; i += 256) {
    const int v = i / FPB, k = i % FPB;
    uint32_t bc = ((uint32_t)v >> (k * NBITS)) & ((1u << NBITS) - 1u);
    bc = bc < (uint32_t)p.pl.nb ? bc : (uint32_t)(p.pl.nb - 1);
    s_lut[i] = p.pl.bw[bc];
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
  // wave index, uniform (so is everything the doc cursor derives from it)
  const int64_t wv = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t g = wv / p.NR, r = wv - g * p.NR;
  if (g >= p.ngroups) return;  // wave-uniform, after the only barrier

  // ---- query block: NSUB queries, token l32 of query g*NSUB+sub in column l32 ----
  u32x4 bq[NSUB][KS];
  float qsc[NSUB];
  const bool f_norm_q = (p.normalize & 1) != 0;
  const bool f_norm_d = (p.normalize & 2) != 0;
#pragma unroll
  for (int sub = 0; sub < NSUB; ++sub) {
    const int64_t q = g * NSUB + sub;
    const bool valid = q < p.q.n && l32 < seq_len(p.q, q);
    const char* rowp = valid ? seq_row0(p.q, q) + (int64_t)l32 * p.q.sl_b : nullptr;
    float ss = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int e = h * HALF + ks * 8;
      bq[sub][ks] = (valid && e < p.q.dim) ? *(const u32x4*)(rowp + (int64_t)e * 2) : (u32x4){0u, 0u, 0u, 0u};
      if (f_norm_q) ss += chunk_sumsq<EK>(bq[sub][ks]);
    }
    ss += __shfl_xor(ss, 32);
    qsc[sub] = valid ? (f_norm_q ? inv_norm(ss) : 1.f) : 0.f;
  }

  // ---- documents [j0, j1) as a stream of 32-token tiles ----
  const int64_t j0 = r * p.R;
  const int64_t j1 = j0 + p.R < p.pl.n ? j0 + p.R : p.pl.n;
  auto dlen = [&](int64_t j) -> int64_t { return doc_len<SRC_PLAID>(p, j); };
  auto dtok = [&](int64_t j) -> int64_t { return p.pl.cu ? (int64_t)p.pl.cu[j] : j * p.pl.codes_sn; };
  auto store = [&](int64_t j, int sub, float v) {
    const int64_t q = g * NSUB + sub;
    if (q < p.q.n)
      ((__attribute__((address_space(1))) float*)p.out)[q * p.osq + j * p.osd] = v;
  };
  // tile descriptor (wave-uniform); j = -1: past the range
  struct Tile {
    int64_t j, tok;
    int t, nv;
  };
  // descriptors are wave-uniform by construction; say so, so the buffer
  // descriptors built from them live in scalar registers
  auto uni64 = [](int64_t x) -> int64_t {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
  };
  auto uni = [&](const Tile& t) -> Tile {
    return Tile{uni64(t.j), uni64(t.tok), __builtin_amdgcn_readfirstlane(t.t), __builtin_amdgcn_readfirstlane(t.nv)};
  };
  // first non-empty doc at or after j (empty docs score 0 on the way)
  auto open_doc = [&](int64_t j) -> Tile {
    while (j < j1) {
      const int64_t len = dlen(j);
      if (len > 0) return uni(Tile{j, dtok(j), 0, (int)(len < 32 ? len : 32)});
      if (lane < NSUB) store(j, lane, 0.f);
      ++j;
    }
    return Tile{-1, 0, 0, 0};
  };
  auto next_tile = [&](const Tile& c) -> Tile {
    if (c.j < 0) return c;
    const int64_t len = dlen(c.j);
    const int64_t start = (int64_t)(c.t + 1) * 32;
    if (start < len) {
      const int64_t rem = len - start;
      return uni(Tile{c.j, c.tok + 32, c.t + 1, (int)(rem < 32 ? rem : 32)});
    }
    return open_doc(c.j + 1);
  };

  const __amdgpu_buffer_rsrc_t rcent = make_rsrc(p.pl.cent, sat_u32(p.pl.ncent * p.pl.cent_sb));
  auto load_code = [&](const Tile& d) -> int32_t {
    if (d.j < 0) return 0;
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(p.pl.codes + d.tok, (uint32_t)d.nv * 4u);
    return (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rc, l32 < d.nv ? (uint32_t)l32 * 4u : kOOB, 0, 0);
  };
  struct Stage {
    u32x4 c[CVL];
    uint32_t rw[RVL];
  };
  auto load_data = [&](const Tile& d, int32_t code, Stage& st) {
    const bool ok = d.j >= 0 && l32 < d.nv;
    int64_t cd = code;
    cd = (cd < 0 || cd >= p.pl.ncent) ? 0 : cd;
    const uint32_t coff = ok ? (uint32_t)(cd * p.pl.cent_sb) + (uint32_t)(h * HALF * CSZ) : kOOB;
#pragma unroll
    for (int v = 0; v < CVL; ++v) st.c[v] = __builtin_amdgcn_raw_buffer_load_b128(rcent, coff == kOOB ? kOOB : coff + 16u * v, 0, 0);
    const __amdgpu_buffer_rsrc_t rres =
        make_rsrc(p.pl.res + (d.j >= 0 ? d.tok : 0) * p.pl.res_st, ok ? sat_u32((int64_t)d.nv * p.pl.res_st) : 0u);
    const uint32_t roff = ok ? (uint32_t)l32 * (uint32_t)p.pl.res_st + (uint32_t)(h * RBL) : kOOB;
#pragma unroll
    for (int v = 0; v < RVL; ++v)
      st.rw[v] = __builtin_amdgcn_raw_buffer_load_b32(rres, roff == kOOB ? kOOB : roff + 4u * v, 0, 0);
  };

  f32x16 acc[NSUB];
  float m[NSUB];
#pragma unroll
  for (int sub = 0; sub < NSUB; ++sub) m[sub] = NEG_INF;

  // decode tile d from st into A fragments, MFMA, running max; doc end: score.
  // Two passes over the lane's half row (the norm needs all of it before any
  // element is scaled): squares first, then the same fp32 values again,
  // scaled, rounded and fed to the MFMA chunk by chunk.
  auto cent_chunk = [&](const Stage& st, int ks, float* cv) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int ei = ks * 8 + e;  // element of this lane's half
      if constexpr (CD == EK_F32) cv[e] = __uint_as_float(st.c[ei >> 2][ei & 3]);
      else if constexpr (CD == EK_BF16)
        cv[e] = (ei & 1) ? bf16hi_to_f32(st.c[ei >> 3][(ei >> 1) & 3]) : bf16lo_to_f32(st.c[ei >> 3][(ei >> 1) & 3]);
      else {
        const uint32_t w = st.c[ei >> 3][(ei >> 1) & 3];
        cv[e] = f16_to_f32((uint16_t)((ei & 1) ? (w >> 16) : (w & 0xffffu)));
      }
    }
  };
  // bucket weights of chunk ks's 8 fields: 8 / FPB residual bytes, one LDS entry each
  auto bw_chunk = [&](const Stage& st, int ks, float* bw) {
#pragma unroll
    for (int b = 0; b < 8 / FPB; ++b) {
      const int byte_i = (ks * 8) / FPB + b;
      const uint32_t byv = (st.rw[byte_i >> 2] >> ((byte_i & 3) * 8)) & 0xffu;
      if constexpr (FPB == 4) {
        const f32x4 t = *(const f32x4*)&s_lut[byv * 4];
#pragma unroll
        for (int k = 0; k < 4; ++k) bw[b * 4 + k] = t[k];
      } else if constexpr (FPB == 2) {
        const float2 t = *(const float2*)&s_lut[byv * 2];
        bw[b * 2] = t.x;
        bw[b * 2 + 1] = t.y;
      } else {
        bw[b] = s_lut[byv];
      }
    }
  };
  auto compute = [&](const Tile& d, const Stage& st) {
    float cs[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      float cv[8], bw[8];
      cent_chunk(st, ks, cv);
      bw_chunk(st, ks, bw);
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = (FULLD || (h * HALF + ks * 8 + e) < p.q.dim) ? cv[e] + bw[e] : 0.f;
        ss = fmaf(x, x, ss);
      }
      cs[ks] = ss;
    }
    // chunk sums in the xor-tree order of the decode kernel's row lanes:
    // pairs, then pairs of pairs, ... within the half, then across halves
#pragma unroll
    for (int w = 1; w < KS; w <<= 1)
#pragma unroll
      for (int c = 0; c < KS; c += 2 * w) cs[c] = cs[c] + cs[c + w];
    float ss = cs[0];
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
      ss = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    const float sc = f_norm_d ? inv_norm(ss) : 1.f;
    // The second pass recomputes the first pass's values on purpose: opaque
    // copies of the staged words keep the compiler from holding all 128
    // intermediate values live between the passes instead.
    Stage s2;
#pragma unroll
    for (int v = 0; v < CVL; ++v) {
      s2.c[v] = st.c[v];
      asm volatile("" : "+v"(s2.c[v]));
    }
#pragma unroll
    for (int v = 0; v < RVL; ++v) {
      s2.rw[v] = st.rw[v];
      asm volatile("" : "+v"(s2.rw[v]));
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      float cv[8], bw[8];
      cent_chunk(s2, ks, cv);
      bw_chunk(s2, ks, bw);
      u32x4 af;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int e0 = h * HALF + ks * 8 + 2 * k;
        const float x0 = (FULLD || e0 < p.q.dim) ? cv[2 * k] + bw[2 * k] : 0.f;
        const float x1 = (FULLD || e0 + 1 < p.q.dim) ? cv[2 * k + 1] + bw[2 * k + 1] : 0.f;
        // bf16: one packed round-to-nearest-even conversion per pair (the
        // fp16 pair conversion would round toward zero: keep the scalar one)
        if constexpr (EK == EK_F16)
          af[k] = f32_to_f16_bits(x0 * sc) | (f32_to_f16_bits(x1 * sc) << 16);
        else
          af[k] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){x0 * sc, x1 * sc}, bf16x2));
      }
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub) acc[sub] = mfma32<EK>(ks == 0 ? f32x16{} : acc[sub], &af, &bq[sub][ks]);
    }
    // running max over the tile's valid rows (row of element e: 8*(e/4) + 4h + e%4)
    if (d.nv == 32) {
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
        for (int e = 0; e < 16; ++e) m[sub] = max_nan(m[sub], acc[sub][e]);
    } else {
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (8 * (e >> 2) + 4 * h + (e & 3) < d.nv) m[sub] = max_nan(m[sub], acc[sub][e]);
    }
    if ((int64_t)(d.t + 1) * 32 >= dlen(d.j)) {
      // doc end: column maxima over both halves, scaled, summed over the
      // query's tokens in column order
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub) {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(m[sub]), __float_as_uint(m[sub]), false, false);
        const float mm = max_nan(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
        const float v = __builtin_isfinite(mm) ? mm * qsc[sub] : 0.f;
        auto col = [&](int c) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), c)); };
        // the tile kernel's flush order: that kernel puts up to 4 queries of
        // <= 32 tokens in one group, query q at place q, and its sum starts at
        // 4-column chunk q % (Lq / 4) and wraps
        float s = 0.f;
        if ((p.LU & 3) == 0) {
          const int nv4 = p.LU >> 2;
          int c = (int)((g * NSUB + sub) % nv4);
          for (int j = 0; j < nv4; ++j) {
            s += col(4 * c);
            s += col(4 * c + 1);
            s += col(4 * c + 2);
            s += col(4 * c + 3);
            c = (c + 1 == nv4) ? 0 : c + 1;
          }
        } else {
          for (int c = 0; c < p.LU; ++c) s += col(c);
        }
        if (lane == 0) store(d.j, sub, s * p.out_scale);
        m[sub] = NEG_INF;
      }
    }
  };

  // pipeline: compute tile c, data of tile c+1 in flight, code of tile c+2 in flight
  Tile tc = open_doc(j0);
  Tile t1 = next_tile(tc);
  Stage sa, sb;
  const int32_t code_c = load_code(tc);
  load_data(tc, code_c, sa);
  int32_t code1 = load_code(t1);
  while (tc.j >= 0) {
    Tile t2 = next_tile(t1);
    load_data(t1, code1, sb);
    int32_t code2 = load_code(t2);
    compute(tc, sa);
    tc = t1;
    t1 = t2;
    code1 = code2;
    if (tc.j < 0) break;
    t2 = next_tile(t1);
    load_data(t1, code1, sa);
    code2 = load_code(t2);
    compute(tc, sb);
    tc = t1;
    t1 = t2;
    code1 = code2;
  }
}

// Gather variant of the stream kernel (same arithmetic, bitwise the same
// scores). Centroid rows and residual bytes go straight from memory into a
// per-wave LDS stage (buffer_load ... lds), 16 lanes per 256-byte row, so
// one load instruction covers 4 whole rows (8 cache lines) instead of 64 half
// rows in 64 lines; the address path, not the memory, bounded the per-lane
// gathers. Each 16-byte chunk of row R sits at slot chunk ^ (R % LPR) so
// that a lane's fragment reads (row l32, chunk h*KS + ks) spread over all
// banks. The decoded fp32 half row stays in VGPRs (no staging registers
// now), so the decode runs once. One LDS stage per wave: tile c is read out
// of it into registers first, then the gather of tile c+1 overwrites it and
// is in flight while tile c is decoded and scored (9 KB of LDS per wave at
// d = 128, 3 waves per SIMD).
//
// Waits are explicit: the compiler does not count the inline-asm gathers,
// so every iteration starts with vmcnt(0) (tile c and code c+1 landed; this
// wave issued nothing since), and the gather of tile c+1 waits for
// lgkmcnt(0) (tile c's LDS reads done). Doc scores are stored one iteration
// late, after the first wait, so a store never holds up a gather.
template <int EK, int DPAD, int CD, int NBITS, bool FULLD, bool SPLIT, int QN>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DPAD >= 128 ? (QN > 1 ? 2 : (SPLIT ? 4 : 3)) : (QN > 1 ? 3 : 4))))
    plaid_gather_kernel(const Params p) {
  using T = KT<EK, DPAD>;
  constexpr int KS = T::KSTEPS;            // 8-element chunks per lane (= MFMA k-steps)
  constexpr int HALF = DPAD / 2;
  constexpr int RB = DPAD * 2;             // centroid row bytes (bf16 / fp16)
  constexpr int LPR = RB / 16;             // gather lanes per row
  constexpr int RPI = 64 / LPR;            // rows per gather instruction
  constexpr int NI = 32 / RPI;             // centroid gather instructions per tile
  constexpr int RSB = DPAD * NBITS / 8;    // residual bytes per (padded) row
  constexpr int NR = (32 * RSB + 1023) / 1024;  // residual gather instructions per tile
  constexpr int RBL = HALF * NBITS / 8;    // residual bytes per lane
  constexpr int RVL = RBL / 4;
  constexpr int FPB = 8 / NBITS;
  constexpr int CBYTES = 32 * RB;
  constexpr int STB = CBYTES + NR * 1024;  // one stage: 32 centroid rows + residual tile
  static_assert(RBL % 4 == 0 && CD != EK_F32, "gather layout");
  static_assert(!SPLIT || CD == EK, "split form feeds stored centroid chunks to the MFMA");
  static_assert(QN == 1 || (SPLIT && QN == 2), "two queries per wavefront in the split form only");
  constexpr float NEG_INF = -__builtin_huge_valf();

  // byte -> bucket weights: fp32 values (exact decode), or for the split
  // form the byte's fields rounded to the MFMA type and packed in pairs
  // (s_lut as uint2 per byte) and the sum of their squares in fp32 (s_r2)
  constexpr int LUTW = SPLIT ? 2 * 256 : FPB * 256;
  __shared__ __attribute__((aligned(16))) float s_lut[LUTW];
  __shared__ __attribute__((aligned(1024))) char s_st[4][STB];
  __shared__ __attribute__((aligned(16))) float s_sc[4][SPLIT ? 32 : 1];
  __shared__ float s_r2[SPLIT ? 256 : 1];
  if constexpr (SPLIT) {
    for (int v = threadIdx.x; v < 256; v += 256) {
      uint32_t h16[4] = {0u, 0u, 0u, 0u};
      float r2 = 0.f;
      for (int k = 0; k < FPB; ++k) {
        uint32_t bc = ((uint32_t)v >> (k * NBITS)) & ((1u << NBITS) - 1u);
        bc = bc < (uint32_t)p.pl.nb ? bc : (uint32_t)(p.pl.nb - 1);
        const float w = p.pl.bw[bc];
        const uint32_t hb = EK == EK_F16 ? f32_to_f16_bits(w) : f32_to_bf16_bits(w);
        const float wr = EK == EK_F16 ? f16_to_f32((uint16_t)hb) : __uint_as_float(hb << 16);
        h16[k] = hb;
        r2 = fmaf(wr, wr, r2);
      }
      uint32_t* e = (uint32_t*)&s_lut[v * 2];
      e[0] = h16[0] | (h16[1] << 16);
      e[1] = h16[2] | (h16[3] << 16);
      s_r2[v] = r2;
    }
  } else {
    for (int i = threadIdx.x; i < 256 * FPB; i += 256) {
      const int v = i / FPB, k = i % FPB;
      uint32_t bc = ((uint32_t)v >> (k * NBITS)) & ((1u << NBITS) - 1u);
      bc = bc < (uint32_t)p.pl.nb ? bc : (uint32_t)(p.pl.nb - 1);
      s_lut[i] = p.pl.bw[bc];
    }
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
  const bool f_norm_d = (p.normalize & 2) != 0;
#pragma unroll
  for (int sub = 0; sub < QN; ++sub) {
    const int64_t q = g * QN + sub;
    const bool valid = q < p.q.n && l32 < seq_len(p.q, q);
    const char* rowp = valid ? seq_row0(p.q, q) + (int64_t)l32 * p.q.sl_b : nullptr;
    float ss = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int e = h * HALF + ks * 8;
      bq[sub][ks] = (valid && e < p.q.dim) ? *(const u32x4*)(rowp + (int64_t)e * 2) : (u32x4){0u, 0u, 0u, 0u};
      if (f_norm_q) ss += chunk_sumsq<EK>(bq[sub][ks]);
    }
    ss += __shfl_xor(ss, 32);
    qsc[sub] = valid ? (f_norm_q ? inv_norm(ss) : 1.f) : 0.f;
  }

  const int64_t j0 = r * p.R;
  const int64_t j1 = j0 + p.R < p.pl.n ? j0 + p.R : p.pl.n;
  auto dlen = [&](int64_t j) -> int64_t { return doc_len<SRC_PLAID>(p, j); };
  auto dtok = [&](int64_t j) -> int64_t { return p.pl.cu ? (int64_t)p.pl.cu[j] : j * p.pl.codes_sn; };
  auto store = [&](int64_t j, int sub, float v) {
    const int64_t q = g * QN + sub;
    if (q < p.q.n) ((__attribute__((address_space(1))) float*)p.out)[q * p.osq + j * p.osd] = v;
  };
  struct Tile {
    int64_t j, tok;
    int t, nv;
  };
  auto uni64 = [](int64_t x) -> int64_t {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
  };
  auto uni = [&](const Tile& t) -> Tile {
    return Tile{uni64(t.j), uni64(t.tok), __builtin_amdgcn_readfirstlane(t.t), __builtin_amdgcn_readfirstlane(t.nv)};
  };
  auto open_doc = [&](int64_t j) -> Tile {
    while (j < j1) {
      const int64_t len = dlen(j);
      if (len > 0) return uni(Tile{j, dtok(j), 0, (int)(len < 32 ? len : 32)});
      if (lane < QN) store(j, lane, 0.f);
      ++j;
    }
    return Tile{-1, 0, 0, 0};
  };
  auto next_tile = [&](const Tile& c) -> Tile {
    if (c.j < 0) return c;
    const int64_t len = dlen(c.j);
    const int64_t start = (int64_t)(c.t + 1) * 32;
    if (start < len) {
      const int64_t rem = len - start;
      return uni(Tile{c.j, c.tok + 32, c.t + 1, (int)(rem < 32 ? rem : 32)});
    }
    return open_doc(c.j + 1);
  };
  auto load_code = [&](const Tile& d) -> int32_t {
    if (d.j < 0) return 0;
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(p.pl.codes + d.tok, (uint32_t)d.nv * 4u);
    return (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rc, l32 < d.nv ? (uint32_t)l32 * 4u : kOOB, 0, 0);
  };
  auto rsrc_words = [](const void* base, uint32_t nbytes) -> u32x4 {
    const uint64_t b = (uint64_t)base;
    return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b),
                 (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32) & 0xffffu),
                 (uint32_t)__builtin_amdgcn_readfirstlane(nbytes), 0x00020000u};
  };
  // rows past the tile's end get offset kInvRow (+ chunk), at or beyond the
  // table's record count (the host keeps tables below kInvRow bytes)
  const u32x4 dcent = rsrc_words(p.pl.cent, (uint32_t)(p.pl.ncent * p.pl.cent_sb));
  auto lds_addr = [&](int off) -> uint32_t {
    return (uint32_t)__builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)(&s_st[wl][0]) + (uint32_t)off);
  };
  auto dma = [&](uint32_t lds, uint32_t voff, const u32x4& desc) {
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
  // gather tile d (code of row l32 in lane l32) into this wave's stage, once
  // the stage's previous contents have been read (lgkmcnt(0))
  auto gather = [&](const Tile& d, int32_t code) {
    if (d.j < 0) return;
    int64_t cd = code;
    cd = (cd < 0 || cd >= p.pl.ncent) ? 0 : cd;
    const uint32_t rowoff = l32 < d.nv ? (uint32_t)cd * (uint32_t)p.pl.cent_sb : kInvRow;
    uint32_t voff[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int row = i * RPI + lane / LPR;
      const int chunk = (lane % LPR) ^ (row % LPR);
      voff[i] = (uint32_t)__builtin_amdgcn_ds_bpermute(row * 4, (int)rowoff) + (uint32_t)(chunk * 16);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int i = 0; i < NI; ++i) dma(lds_addr(i * 1024), voff[i], dcent);
    const u32x4 dres = rsrc_words(p.pl.res + d.tok * p.pl.res_st, (uint32_t)d.nv * (uint32_t)p.pl.res_st);
#pragma unroll
    for (int i = 0; i < NR; ++i) dma(lds_addr(CBYTES + i * 1024), (uint32_t)(i * 1024 + lane * 16), dres);
  };

  float m[QN], pend_v[QN];
  int rot0[QN];  // first 4-column chunk of each query's flush order (loop-invariant)
#pragma unroll
  for (int sub = 0; sub < QN; ++sub) {
    m[sub] = NEG_INF;
    pend_v[sub] = 0.f;
    rot0[sub] = (p.LU & 3) == 0 ? (int)((g * QN + sub) % (p.LU >> 2)) : 0;
  }
  int64_t pend_j = -1;

  // tile data of this wave's stage into registers
  struct Regs {
    u32x4 cw[KS];
    uint32_t rw[RVL];
  };
  auto read_stage = [&](Regs& rg) {
    const char* stage = &s_st[wl][0];
    const char* rp = stage + CBYTES + l32 * (int)p.pl.res_st + h * RBL;
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
    for (int ks = 0; ks < KS; ++ks) {
      const int cc = h * KS + ks;
      rg.cw[ks] = *(const u32x4*)(stage + l32 * RB + ((cc ^ (l32 % LPR)) * 16));
    }
  };
  // split form: x = c + r with c the stored centroid chunk and r the bucket
  // weights rounded to the MFMA type; q.x = q.c + q.r (two MFMA chains into
  // one accumulator), ||x||^2 = ||c||^2 + 2 c.r + ||r||^2 (dot2 on the
  // packed pairs, byte sums of r^2 from the table), and the row scale is
  // applied to the accumulator instead of to every element.
  // (the normalise flag stays a runtime branch: compiling both loop bodies
  // into one straight block raised register pressure past 128 VGPRs)
  auto compute_split = [&](const Tile& d, const Regs& rg, f32x16* acc) {
    const uint32_t* rw = rg.rw;
    float cc = 0.f, cr = 0.f, r2 = 0.f;
    auto byte_at = [&](int byte_i) -> uint32_t { return (rw[byte_i >> 2] >> ((byte_i & 3) * 8)) & 0xffu; };
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const bool live = FULLD || (h * HALF + ks * 8) < p.q.dim;  // chunks are whole: dim % 8 == 0
      u32x4 rv;
      float rs = 0.f;
      if constexpr (FPB == 4) {
        const uint32_t b0 = byte_at(2 * ks), b1 = byte_at(2 * ks + 1);
        const uint2 e0 = *(const uint2*)&s_lut[b0 * 2];
        const uint2 e1 = *(const uint2*)&s_lut[b1 * 2];
        rv = u32x4{e0.x, e0.y, e1.x, e1.y};
        rs = s_r2[b0] + s_r2[b1];
      } else if constexpr (FPB == 2) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t b = byte_at(4 * ks + k);
          rv[k] = *(const uint32_t*)&s_lut[b * 2];
          rs += s_r2[b];
        }
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t b0 = byte_at(8 * ks + 2 * k), b1 = byte_at(8 * ks + 2 * k + 1);
          rv[k] = (*(const uint32_t*)&s_lut[b0 * 2] & 0xffffu) | (*(const uint32_t*)&s_lut[b1 * 2] << 16);
          rs += s_r2[b0] + s_r2[b1];
        }
      }
      const u32x4 z = {0u, 0u, 0u, 0u};
      const u32x4 ca = live ? rg.cw[ks] : z;
      const u32x4 ra = live ? rv : z;
      r2 += live ? rs : 0.f;
      if (f_norm_d) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          cc = dot2<EK>(ca[w], ca[w], cc);
          cr = dot2<EK>(ca[w], ra[w], cr);
        }
      }
#pragma unroll
      for (int sub = 0; sub < QN; ++sub) {
        acc[sub] = mfma32<EK>(ks == 0 ? f32x16{} : acc[sub], &ca, &bq[sub][ks]);
        acc[sub] = mfma32<EK>(acc[sub], &ra, &bq[sub][ks]);
      }
    }
    // row l32's scale to the
    // accumulator layout: element i of lane l is row 8 (i / 4) + 4 h + i % 4
    float sc = 1.f;
    if (f_norm_d) {
      float ss = fmaf(2.f, cr, cc) + r2;
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
      ss = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
      sc = __builtin_amdgcn_rsqf(fmaxf(ss, 1e-24f));  // 1 / max(||x||, 1e-12)
    }
    if (h == 0) s_sc[wl][l32] = sc;
    // rows past the tile's end are set to -inf by a select (in partial tiles
    // only): their staged data is not the tile's and may hold NaN, which an
    // added -inf bias would keep
    const bool part = d.nv < 32;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 sc4 = *(const f32x4*)&s_sc[wl][8 * j + 4 * h];
#pragma unroll
      for (int sub = 0; sub < QN; ++sub)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float v = acc[sub][4 * j + t] * sc4[t];
          acc[sub][4 * j + t] = (part && 8 * j + 4 * h + t >= d.nv) ? NEG_INF : v;
        }
    }
  };
  auto compute = [&](const Tile& d, const Regs& rg) {
    f32x16 acc[QN];
    if constexpr (SPLIT) {
      compute_split(d, rg, acc);
    } else {
    const uint32_t* rw = rg.rw;
    float x[KS][8];
    float cs[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const u32x4 cw = rg.cw[ks];
      float bw[8];
#pragma unroll
      for (int b = 0; b < 8 / FPB; ++b) {
        const int byte_i = (ks * 8) / FPB + b;
        const uint32_t byv = (rw[byte_i >> 2] >> ((byte_i & 3) * 8)) & 0xffu;
        if constexpr (FPB == 4) {
          const f32x4 t = *(const f32x4*)&s_lut[byv * 4];
#pragma unroll
          for (int k = 0; k < 4; ++k) bw[b * 4 + k] = t[k];
        } else if constexpr (FPB == 2) {
          const float2 t = *(const float2*)&s_lut[byv * 2];
          bw[b * 2] = t.x;
          bw[b * 2 + 1] = t.y;
        } else {
          bw[b] = s_lut[byv];
        }
      }
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t w = cw[e >> 1];
        float c;
        if constexpr (CD == EK_BF16) c = (e & 1) ? bf16hi_to_f32(w) : bf16lo_to_f32(w);
        else c = f16_to_f32((uint16_t)((e & 1) ? (w >> 16) : (w & 0xffffu)));
        const float xv = (FULLD || (h * HALF + ks * 8 + e) < p.q.dim) ? c + bw[e] : 0.f;
        x[ks][e] = xv;
        ss = fmaf(xv, xv, ss);
      }
      cs[ks] = ss;
    }
#pragma unroll
    for (int w = 1; w < KS; w <<= 1)
#pragma unroll
      for (int c = 0; c < KS; c += 2 * w) cs[c] = cs[c] + cs[c + w];
    float ss = cs[0];
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
      ss = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    const float sc = f_norm_d ? inv_norm(ss) : 1.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 af;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float x0 = x[ks][2 * k] * sc, x1 = x[ks][2 * k + 1] * sc;
        if constexpr (EK == EK_F16)
          af[k] = f32_to_f16_bits(x0) | (f32_to_f16_bits(x1) << 16);
        else
          af[k] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){x0, x1}, bf16x2));
      }
      acc[0] = mfma32<EK>(ks == 0 ? f32x16{} : acc[0], &af, &bq[0][ks]);
    }
    }
#pragma unroll
    for (int sub = 0; sub < QN; ++sub) {
      if (SPLIT || d.nv == 32) {  // split form: rows past the end are already -inf
#pragma unroll
        for (int e = 0; e < 16; ++e) m[sub] = max_nan(m[sub], acc[sub][e]);
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (8 * (e >> 2) + 4 * h + (e & 3) < d.nv) m[sub] = max_nan(m[sub], acc[sub][e]);
      }
    }
    if ((int64_t)(d.t + 1) * 32 >= dlen(d.j)) {
#pragma unroll
     for (int sub = 0; sub < QN; ++sub) {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(m[sub]), __float_as_uint(m[sub]), false, false);
      const float mm = max_nan(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
      const float v = __builtin_isfinite(mm) ? mm * qsc[sub] : 0.f;
      auto col = [&](int c) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), c)); };
      // the tile kernel's flush order (query g at place g of its group of 4:
      // the sum starts at 4-column chunk g % (Lq / 4) and wraps)
      float s = 0.f;
      if ((p.LU & 3) == 0) {
        const int nv4 = p.LU >> 2;
        int c = rot0[sub];
        for (int j = 0; j < nv4; ++j) {
          s += col(4 * c);
          s += col(4 * c + 1);
          s += col(4 * c + 2);
          s += col(4 * c + 3);
          c = (c + 1 == nv4) ? 0 : c + 1;
        }
      } else {
        for (int c = 0; c < p.LU; ++c) s += col(c);
      }
      pend_v[sub] = s * p.out_scale;
      m[sub] = NEG_INF;
     }
      pend_j = d.j;
    }
  };

  Tile tc = open_doc(j0);
  Tile t1 = next_tile(tc);
  const int32_t code_c = load_code(tc);
  int32_t code1 = load_code(t1);
  asm volatile("s_waitcnt vmcnt(0)" : "+v"(code1) : : "memory");
  gather(tc, code_c);
  while (tc.j >= 0) {
    const Tile t2 = next_tile(t1);
    // tile tc's gather and code1 have landed
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(code1) : : "memory");
    if (pend_j >= 0) {
      if (lane == 0)
#pragma unroll
        for (int sub = 0; sub < QN; ++sub) store(pend_j, sub, pend_v[sub]);
      pend_j = -1;
    }
    Regs rg;
    read_stage(rg);
    gather(t1, code1);
    code1 = load_code(t2);
    compute(tc, rg);
    tc = t1;
    t1 = t2;
  }
  if (pend_j >= 0 && lane == 0)
#pragma unroll
    for (int sub = 0; sub < QN; ++sub) store(pend_j, sub, pend_v[sub]);
  // no gather may still be writing this wave's LDS when it exits
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

template <int EK, int DPAD, int CD, int NBITS>
int launch_stream_nsub(int nsub, const Params& p, int64_t nblocks, hipStream_t s) {
  if (nsub != 1 && !(nsub == 2 && p.gather == 2)) return LIK_ERR_UNSUPPORTED;
  if (p.gather) {
    const bool full = p.q.dim == DPAD;
    auto go = [&](auto kern) {
      launch_kernel(kern, dim3((unsigned)nblocks), dim3(256), 0, s, p);
      return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
    };
    if constexpr (CD == EK) {
      if (p.gather == 2 && nsub == 2)
        return full ? go(plaid_gather_kernel<EK, DPAD, CD, NBITS, true, true, 2>)
                    : go(plaid_gather_kernel<EK, DPAD, CD, NBITS, false, true, 2>);
      if (p.gather == 2)
        return full ? go(plaid_gather_kernel<EK, DPAD, CD, NBITS, true, true, 1>)
                    : go(plaid_gather_kernel<EK, DPAD, CD, NBITS, false, true, 1>);
    }
    return full ? go(plaid_gather_kernel<EK, DPAD, CD, NBITS, true, false, 1>)
                : go(plaid_gather_kernel<EK, DPAD, CD, NBITS, false, false, 1>);
  }
  if (p.q.dim == DPAD)
    launch_kernel(plaid_stream_kernel<EK, DPAD, CD, NBITS, 1, true>, dim3((unsigned)nblocks), dim3(256), 0, s, p);
  else
    launch_kernel(plaid_stream_kernel<EK, DPAD, CD, NBITS, 1, false>, dim3((unsigned)nblocks), dim3(256), 0, s, p);
  return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
}

template <int EK, int DPAD, int CD>
int launch_stream_nbits(int nbits, int nsub, const Params& p, int64_t nblocks, hipStream_t s) {
  switch (nbits) {
    case 2: return launch_stream_nsub<EK, DPAD, CD, 2>(nsub, p, nblocks, s);
    case 4: return launch_stream_nsub<EK, DPAD, CD, 4>(nsub, p, nblocks, s);
    case 8: return launch_stream_nsub<EK, DPAD, CD, 8>(nsub, p, nblocks, s);
    default: return LIK_ERR_UNSUPPORTED;
  }
}

template <int EK, int DPAD>
int launch_stream_cd(int cd, int nbits, int nsub, const Params& p, int64_t nblocks, hipStream_t s) {
  switch (cd) {
    case EK_BF16: return launch_stream_nbits<EK, DPAD, EK_BF16>(nbits, nsub, p, nblocks, s);
    case EK_F16: return launch_stream_nbits<EK, DPAD, EK_F16>(nbits, nsub, p, nblocks, s);
    default: return LIK_ERR_UNSUPPORTED;
  }
}

// Launch the stream kernel: p.ngroups query groups of nsub queries, p.NR doc
// ranges of p.R docs each, one wavefront per (group, range), 4 per block.
int launch_plaid_stream(int ek, int cd, int dpad, int nsub, const Params& p, hipStream_t s) {
  const int64_t waves = p.ngroups * p.NR;
  const int64_t nblocks = (waves + 3) / 4;
  if (nblocks > 0x7fffffffLL) return LIK_ERR_UNSUPPORTED;
  const int nbits = p.pl.nbits;
  if (ek == EK_BF16) {
    if (dpad == 64) return launch_stream_cd<EK_BF16, 64>(cd, nbits, nsub, p, nblocks, s);
    if (dpad == 128) return launch_stream_cd<EK_BF16, 128>(cd, nbits, nsub, p, nblocks, s);
  } else {
    if (dpad == 64) return launch_stream_cd<EK_F16, 64>(cd, nbits, nsub, p, nblocks, s);
    if (dpad == 128) return launch_stream_cd<EK_F16, 128>(cd, nbits, nsub, p, nblocks, s);
  }
  return LIK_ERR_UNSUPPORTED;
}

}  // namespace lik
