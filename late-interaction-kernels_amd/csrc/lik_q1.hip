// MaxSim for launches with one 32-column block per group (W = 1, NSUB = 1
// plans: the KD layout, where every query scores its own K docs, and calls
// with one short query): a streaming kernel, one independent wavefront per
// (group, doc range), four per workgroup, no barriers.
//
// With a single column block a doc tile is used by one wavefront only, and
// the work is HBM-bound: what matters is that the loads are coalesced and
// that enough of them are in flight. Each wavefront keeps two 8 KB tiles in
// flight in an LDS ring of its own, loaded by non-temporal buffer_load ...
// lds (M0 saved and restored): with 256-byte rows (d 128), instruction i of
// a tile covers rows 4i .. 4i+3, lane L the 16-byte chunk
// j = (L % 16 - 4 (L / 16) - i) mod 16 of row 4i + L / 16, so an instruction
// reads 1 KB of consecutive rows (8 cache lines; a lane per half row would
// touch 32) and lands it at LDS offset 1024 i + 16 L. The rotation by
// 4 (row % 4) + row / 4 makes the A-fragment reads (lane (r, h) reads chunk
// 8 h + ks of row r) conflict-free. 128-byte rows (d 64) take 8 rows per
// instruction and the rotation (row % 8) / 2 + 4 (row / 8) mod 8. A tile's fragments go to
// registers first, then the next DMA reuses its slot, so two tiles stay in
// flight during the MFMAs. Everything in the loop that touches vector
// memory is a DMA load (8 per tile), so one fixed vmcnt per tile waits for
// exactly the tile being scored; doc scores are kept in LDS and written
// after the loop. Rows past a doc's end are outside the buffer range (read
// as 0) and masked to -inf before the running max; dims past d read as 0.
//
// Scores are bitwise those of the tile kernel: the same MFMA sequence per
// tile (k-steps in order from a zero accumulator), the max over rows is
// exact, and a doc's column maxima are summed in the tile kernel's flush
// order (4-column chunks from chunk t % (LU / 4) on for unit t of the group,
// or columns in order when LU % 4 != 0).
//
// Reference semantics: autograd.py:356-461 / reference.py:26-98 (MaxSim with
// prefix masks and the KD layout), varlen.py:452-493 (packed docs).
#include "lik_kernel.h"

namespace lik {

constexpr int kQ1RMax = 128;  // docs per wavefront (the host routes larger R to the tile kernel)
constexpr int kQ1Scores = 256;  // doc scores per wavefront held until the loop ends (docs x units)

// two workgroups per CU (their LDS rings take 2 x 64 KB): two waves per SIMD
// EXT (256-byte rows): with p.amax (the training forward) also the winner
// doc-token index per (query token, doc), and with p.normalize & 2 the doc
// rows L2-normalised in registers before their MFMAs, bitwise as the tile
// kernel does it (a row's 16 chunk sums of squares added as a balanced tree
// in chunk order: each lane holds chunks 0..7 or 8..15 of its row, the two
// halves meet by one lane swap; scaled in fp32 and rounded once).
template <int EK, int DPAD, bool FULLD, bool NORMQ, bool EXT = false>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) maxsim_q1_kernel(const Params p) {
  using T = KT<EK, DPAD>;
  constexpr int KS = T::KSTEPS;
  static_assert(T::FRAG_V == 1 && !T::SPLIT && T::IN_B == 2 && DPAD >= 64 && DPAD <= 512, "16-bit rows");
  static_assert(!EXT || DPAD == 128, "argmax and doc normalise take 256-byte rows");
  // The ring moves units of 32 rows: a whole tile for rows of <= 256 bytes;
  // wider rows (d 256, 512) are split into NU units of 256 bytes per row,
  // unit c holding bytes [128 c, 128 c + 128) of each half row, which are
  // the A fragments of k-steps 8c .. 8c + 7. One DMA instruction moves 1 KB:
  // RPI rows of CPR 16-byte chunks; a unit takes NI instructions.
  constexpr int NU = DPAD >= 256 ? DPAD / 128 : 1;
  constexpr int KSU = KS / NU;  // k-steps per unit
  constexpr int CPR = NU > 1 ? 16 : DPAD * 2 / 16, RPI = 16 * 4 / CPR, NI = 32 / RPI, TB = NI * 1024;
  constexpr float NEG_INF = -__builtin_huge_valf();
  __shared__ int32_t s_len[4][kQ1RMax];   // doc length (0: empty or not in this launch)
  __shared__ int64_t s_off[4][kQ1RMax];   // byte offset of the doc's token 0
  // doc scores, written to memory after the loop: a store in the loop would
  // make the compiler's load counting wait for tiles still in flight
  __shared__ float s_score[4][kQ1Scores];
  // per-wave ring of two 8 KB tiles (chunks rotated as described above)
  __shared__ __attribute__((aligned(1024))) char s_ring[4][2][TB];

  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
  const int wl = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t item = (int64_t)blockIdx.x * 4 + wl;
  const int64_t g = item / p.NR, r = item - g * p.NR;
  if (g >= p.ngroups) return;  // wave-uniform; the kernel has no barrier

  const int64_t jl0 = r * (int64_t)p.R;
  const int64_t jl1 = (jl0 + p.R < p.ndocs_pg) ? jl0 + p.R : p.ndocs_pg;
  const int nloc = (int)(jl1 - jl0);
  const int64_t kd_base = p.kd_K ? (g / p.nc) * p.kd_K : 0;  // KD: one query per group

  // ---- this group's query tokens as the B fragments of column l32 ----
  u32x4 bq[KS];
  float qsc = 1.f;
  {
    const int col = l32;
    const int ul = col / p.LU;
    const int s = col - ul * p.LU;
    const int64_t u = g * p.QPG + ul;
    bool valid = ul < p.QPG && u < p.nunits;
    const int64_t q = u / p.nc;
    const int64_t tok = (u - q * p.nc) * (int64_t)p.LU + s;
    const char* rowp = nullptr;
    if (valid) {
      valid = tok < seq_len(p.q, q);
      if (valid && p.q.mask) valid = p.q.mask[q * p.q.msn + tok * p.q.msl] != 0;
      rowp = seq_row0(p.q, q) + tok * p.q.sl_b;
    }
    float ss = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int e = h * (DPAD / 2) + ks * T::FE;
      bq[ks] = (valid && (FULLD || e < p.q.dim)) ? *(const u32x4*)(rowp + (int64_t)e * T::IN_B)
                                                 : (u32x4){0u, 0u, 0u, 0u};
      if constexpr (NORMQ) ss += chunk_sumsq<EK>(bq[ks]);
    }
    if constexpr (NORMQ) {
      ss += __shfl_xor(ss, 32);
      qsc = valid ? inv_norm(ss) : 0.f;
    }
    // complete these loads here: pending in the compiler's view at the loop,
    // they would put a full vmcnt(0) in front of the first tile
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(bq[ks]));
  }

  // ---- doc table of this wavefront's range (empty docs score 0 here) ----
  for (int k = lane; k < nloc; k += 64) {
    const int64_t dg = kd_base + jl0 + k;
    const int64_t L = doc_len<SRC_DENSE>(p, dg);
    const bool skip = p.doc_filter == 1 && p.holes != nullptr && p.holes[dg] != 0;
    s_len[wl][k] = skip ? 0 : (int32_t)L;
    s_off[wl][k] = p.d.cu ? (int64_t)p.d.cu[dg] * p.d.sl_b : dg * p.d.sn_b;
    if (L == 0 && !skip) {
      for (int t = 0; t < p.QPG; ++t) {
        const int64_t u = g * p.QPG + t;
        if (u < p.nunits) p.out[u * p.osq + (jl0 + k) * p.osd] = 0.f;
      }
    }
  }
  __builtin_amdgcn_wave_barrier();
  const float osc = p.out_scale;

  // DMA lane offsets of instruction i (row RPI i + L / CPR, chunk rotated
  // by rot(a, i)) and A-fragment LDS offsets of k-step ks of a unit. The
  // rotation gives the 16 lanes of a fragment-read pass 16 different bank
  // groups: (4a + i) mod 16 for 256-byte unit rows (a = row % 4,
  // i = row / 4), (a / 2 + 4i) mod 8 for 128-byte rows (a = row % 8).
  // Chunk j of a unit row is byte chunkb(j) + 128 c of the doc row.
  auto rot = [](int a, int i) { return CPR == 16 ? (4 * a + i) & 15 : ((a >> 1) + 4 * i) & 7; };
  auto chunkb = [](int j) { return NU > 1 && j >= 8 ? DPAD + 16 * (j - 8) : 16 * j; };
  const uint32_t sl = (uint32_t)p.d.sl_b;
  uint32_t drow[NI], dchunk[NI], aoff[KSU];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int a = lane / CPR, j = ((lane % CPR) - rot(a, i)) & (CPR - 1);
    drow[i] = (uint32_t)(RPI * i + a) * sl;
    dchunk[i] = (uint32_t)chunkb(j);
  }
#pragma unroll
  for (int ks = 0; ks < KSU; ++ks) {
    const int i = l32 / RPI, a = l32 % RPI, j = (CPR / 2) * h + ks;
    aoff[ks] = (uint32_t)(i * 1024 + a * (CPR * 16) + ((j + rot(a, i)) & (CPR - 1)) * 16);
  }
  const uint32_t ring_lds = (uint32_t)__builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)(&s_ring[wl][0][0]));

  // ---- cursor: unit c of tile t of local doc k (k == nloc: past the range) ----
  struct Cur {
    int k, t, len;
    int64_t off;
  };
  auto cur_doc = [&](Cur& c, int k) {
    while (k < nloc && s_len[wl][k] == 0) ++k;
    c.k = k;
    c.t = 0;
    c.len = k < nloc ? __builtin_amdgcn_readfirstlane(s_len[wl][k]) : 0;
    const int64_t o = k < nloc ? s_off[wl][k] : 0;
    c.off = (int64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)o) |
            ((int64_t)__builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)o >> 32)) << 32);
  };
  struct Desc {
    int nv, k, t;  // valid rows, local doc, tile of the doc
    bool docend;   // last unit of the doc's last tile
  };
  // DMA of unit CU of the cursor's tile into ring slot S (exactly NI load
  // instructions, whether or not the tile exists); after the tile's last
  // unit the cursor advances
  auto fetch = [&](auto SS, auto CC, Cur& c) -> Desc {
    constexpr int S = decltype(SS)::value, CU = decltype(CC)::value;
    Desc d;
    const int rem = c.len - 32 * c.t;
    d.nv = rem < 32 ? rem : 32;
    d.k = c.k;
    d.t = c.t;
    const bool tile_end = c.len > 0 && rem <= 32;
    d.docend = tile_end && CU == NU - 1;
    // the buffer covers rows [32 t, len) of the doc: later rows read 0
    const uint64_t base = (uint64_t)(p.d.data + c.off) + (uint64_t)((uint32_t)c.t * 32u * sl);
    const uint32_t span = d.nv > 0 ? (uint32_t)(d.nv - 1) * sl + (uint32_t)(p.d.dim * T::IN_B) : 0u;
    const u32x4 desc = {(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)base),
                        (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(base >> 32) & 0xffffu),
                        (uint32_t)__builtin_amdgcn_readfirstlane(span), 0x00020000u};
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const uint32_t cb = dchunk[i] + (uint32_t)(128 * CU);
      // dims past d: out of range
      const uint32_t voff = (FULLD || cb / 2 < (uint32_t)p.d.dim) ? drow[i] + cb : kOOB;
      uint32_t saved;
      asm volatile(
          "s_mov_b32 %0, m0\n\t"
          "s_mov_b32 m0, %1\n\t"
          "s_nop 0\n\t"  // an M0 write needs one wait state before an LDS DMA reads it
          "buffer_load_dwordx4 %2, %3, 0 offen nt lds\n\t"
          "s_mov_b32 m0, %0"
          : "=&s"(saved)
          : "s"(ring_lds + (uint32_t)(S * TB + i * 1024)), "v"(voff), "s"(desc)
          : "memory");
    }
    if (CU == NU - 1) {
      if (tile_end)
        cur_doc(c, c.k + 1);
      else
        c.t += 1;
    }
    return d;
  };

  float m = NEG_INF;
  int mi = -1;  // argmax: doc-token index of m (-1: no valid token yet)
  // a doc ends: column maxima (max over lanes l, l ^ 32) summed per unit in
  // the tile kernel's flush order, written by lane 0
  auto doc_end = [&](int k) {
    if (EXT && p.amax) {
      // winner over lanes l, l ^ 32 (larger value; equal values: lower
      // index), at argmax[(q * docs + j) * Lq + token], -1 for a non-finite max
      const auto sv = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
      const auto si = __builtin_amdgcn_permlane32_swap((uint32_t)mi, (uint32_t)mi, false, false);
      const float v0 = __uint_as_float(sv[0]), v1 = __uint_as_float(sv[1]);
      const int i0 = (int)si[0], i1 = (int)si[1];
      const bool take1 = v1 > v0 || (v1 == v0 && (unsigned)i1 < (unsigned)i0);
      const int win = take1 ? i1 : i0;
      const int ul = l32 / p.LU;
      if (h == 0 && ul < p.QPG) {
        const int64_t u = g * p.QPG + ul;
        const int64_t q = u / p.nc;
        const int64_t tok = p.q_tok0 + (u - q * p.nc) * p.LU + (l32 - ul * p.LU);
        if (u < p.nunits && tok < p.amax_ld)
          p.amax[(q * p.amax_qs + jl0 + k) * p.amax_ld + tok] = __builtin_isfinite(max_nan(v0, v1)) ? win : -1;
      }
      mi = -1;
    }
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    const float mm = max_nan(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    const float v = __builtin_isfinite(mm) ? (NORMQ ? mm * qsc : mm) : 0.f;
    auto col = [&](int c) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), c)); };
    for (int t = 0; t < p.QPG; ++t) {
      const int64_t u = g * p.QPG + t;
      if (u >= p.nunits) break;
      float sum = 0.f;
      if ((p.LU & 3) == 0) {
        const int nv4 = p.LU >> 2;
        int c = t % nv4;
        for (int j = 0; j < nv4; ++j) {
          const int c0 = t * p.LU + 4 * c;
          sum += col(c0);
          sum += col(c0 + 1);
          sum += col(c0 + 2);
          sum += col(c0 + 3);
          c = (c + 1 == nv4) ? 0 : c + 1;
        }
      } else {
        for (int j = 0; j < p.LU; ++j) sum += col(t * p.LU + j);
      }
      if (lane == 0) s_score[wl][k * p.QPG + t] = sum * osc;
    }
    m = NEG_INF;
  };
  // unit CU in slot S: wait for it, read its A fragments, hand the slot to
  // the next fetch (two units on, unit CN), then its MFMAs; the tile's last
  // unit ends with the running max (and the doc's end)
  f32x16 acc;
  auto step = [&](auto SS, auto CC, auto CN, const Desc& d, Cur& c) -> Desc {
    constexpr int S = decltype(SS)::value, CU = decltype(CC)::value;
    // the unit after this one (NI loads) may still be in flight
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(NI) : "memory");
    u32x4 af[KSU];
    const char* slot = (const char*)&s_ring[wl][S][0];
#pragma unroll
    for (int ks = 0; ks < KSU; ++ks) af[ks] = *(const u32x4*)(slot + aoff[ks]);
    // the fragments are in registers before the DMA overwrites the slot
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const Desc dn = fetch(SS, CN, c);
    if constexpr (EXT) {
      if (p.normalize & 2) {
        float cs[KSU];
#pragma unroll
        for (int ks = 0; ks < KSU; ++ks) cs[ks] = chunk_sumsq<EK>(af[ks]);
#pragma unroll
        for (int w = 1; w < KSU; w <<= 1)
#pragma unroll
          for (int c0 = 0; c0 < KSU; c0 += 2 * w) cs[c0] = cs[c0] + cs[c0 + w];
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(cs[0]), __float_as_uint(cs[0]), false, false);
        const float sc = inv_norm(__uint_as_float(sw[0]) + __uint_as_float(sw[1]));
#pragma unroll
        for (int ks = 0; ks < KSU; ++ks)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t v = af[ks][e];
            if constexpr (EK == EK_BF16)
              af[ks][e] = f32_to_bf16_bits(bf16lo_to_f32(v) * sc) | (f32_to_bf16_bits(bf16hi_to_f32(v) * sc) << 16);
            else
              af[ks][e] = f32_to_f16_bits(f16_to_f32((uint16_t)(v & 0xffffu)) * sc) |
                          (f32_to_f16_bits(f16_to_f32((uint16_t)(v >> 16)) * sc) << 16);
          }
      }
    }
#pragma unroll
    for (int ks = 0; ks < KSU; ++ks)
      acc = mfma32<EK>(CU == 0 && ks == 0 ? f32x16{} : acc, &af[ks], &bq[CU * KSU + ks]);
    if constexpr (CU == NU - 1) {
      // element e is row 8 (e / 4) + 4 h + e % 4
      if (d.nv < 32) {
        const int lim = d.nv - 4 * h;
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (8 * (e >> 2) + (e & 3) >= lim) acc[e] = NEG_INF;
      }
      if (EXT && p.amax) {
        // rows in increasing order; only a strictly larger value replaces
        // the winner, so ties keep the lowest doc-token index
        const int r0 = 32 * d.t + 4 * h;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          mi = acc[e] > m ? r0 + 8 * (e >> 2) + (e & 3) : mi;
          m = max_nan(m, acc[e]);  // a NaN row makes the max NaN (scored 0, argmax -1)
        }
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) m = max_nan(m, acc[e]);
      }
      if (d.docend) doc_end(d.k);
    }
    return dn;
  };

  Cur cur;
  cur_doc(cur, 0);
  if (cur.k >= nloc) return;  // (empty docs were written above)
  // Units u, u + 1 in flight (slots u % 2); the loop body is unrolled over
  // U units so slots and unit indices are compile-time. A unit past the
  // range (nv 0) loads nothing and ends the loop.
  constexpr int U = NU > 2 ? NU : 2;
  // (the prologue's stores and query loads complete before the fixed counts start)
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  Desc q0 = fetch(I0{}, I0{}, cur);
  Desc q1 = fetch(I1{}, std::integral_constant<int, 1 % NU>{}, cur);
  bool run = true;
  auto one = [&](auto SI) {
    constexpr int s = decltype(SI)::value;
    if (!run) return;
    const Desc qn = step(std::integral_constant<int, s % 2>{}, std::integral_constant<int, s % NU>{},
                         std::integral_constant<int, (s + 2) % NU>{}, q0, cur);
    if (q1.nv <= 0) {
      run = false;
      return;
    }
    q0 = q1;
    q1 = qn;
  };
  while (run) {
    one(std::integral_constant<int, 0>{});
    one(std::integral_constant<int, 1>{});
    if constexpr (U > 2) {
      one(std::integral_constant<int, 2>{});
      one(std::integral_constant<int, 3>{});
    }
  }
  // no DMA may still be writing this wave's LDS (tiles past the range load nothing)
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __builtin_amdgcn_wave_barrier();
  for (int i = lane; i < nloc * p.QPG; i += 64) {
    const int k = i / p.QPG, t = i - k * p.QPG;
    const int64_t u = g * p.QPG + t;
    if (u < p.nunits && s_len[wl][k] > 0) p.out[u * p.osq + (jl0 + k) * p.osd] = s_score[wl][i];
  }
}

template <int EK, int DPAD>
int launch_q1_t(const Params& p, bool normq, hipStream_t s) {
  if constexpr (DPAD == 128) {
    if (p.amax || (p.normalize & 2)) {
      const int64_t waves = p.ngroups * p.NR;
      const int64_t nb = (waves + 3) / 4;
      if (nb <= 0) return LIK_OK;
      if (nb > 0x7fffffffLL) return LIK_ERR_UNSUPPORTED;
      auto go = [&](auto kern) {
        launch_kernel(kern, dim3((unsigned)nb), dim3(256), 0, s, p);
        return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
      };
      const bool full = p.d.dim == DPAD && p.q.dim == DPAD;
      if (full)
        return normq ? go(maxsim_q1_kernel<EK, DPAD, true, true, true>) : go(maxsim_q1_kernel<EK, DPAD, true, false, true>);
      return normq ? go(maxsim_q1_kernel<EK, DPAD, false, true, true>) : go(maxsim_q1_kernel<EK, DPAD, false, false, true>);
    }
  }
  if (p.amax || (p.normalize & 2)) return LIK_ERR_UNSUPPORTED;
  const int64_t waves = p.ngroups * p.NR;
  const int64_t nb = (waves + 3) / 4;
  if (nb <= 0) return LIK_OK;
  if (nb > 0x7fffffffLL) return LIK_ERR_UNSUPPORTED;
  const bool full = p.d.dim == DPAD && p.q.dim == DPAD;
  auto go = [&](auto kern) {
    launch_kernel(kern, dim3((unsigned)nb), dim3(256), 0, s, p);
    return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
  };
  if (full)
    return normq ? go(maxsim_q1_kernel<EK, DPAD, true, true>) : go(maxsim_q1_kernel<EK, DPAD, true, false>);
  return normq ? go(maxsim_q1_kernel<EK, DPAD, false, true>) : go(maxsim_q1_kernel<EK, DPAD, false, false>);
}

// Docs per wavefront: about 2048 wavefronts (two per SIMD, the kernel's
// occupancy) over the launch, at most kQ1RMax; the tile kernel's choice
// aims at workgroups of several waves and leaves too few wavefronts here.
int q1_docs_per_wave(const Params& p) {
  int64_t R = (p.ndocs_pg * p.ngroups + 2047) / 2048;
  R = R < 1 ? 1 : R;
  return (int)(R > kQ1RMax ? kQ1RMax : R);
}

// Routed here: 16-bit dense scoring in which one 32-column block holds the
// columns of a group as planned (W = 1 plans, the KD layout) or of the
// call's only group (a one-query call whose plan is wider), with nothing in
// the tile loop beyond the plain max (no doc mask holes, token scales, pair
// lists or query-chunk accumulation; doc normalisation and argmax at
// 256-byte rows only), unless the caller forced a column block of several
// waves (lik_launch_opts_t). (Two
// and four blocks per wavefront for queries of up to 128 tokens measured
// slower than the tile kernel's four waves sharing a tile.)
bool q1_eligible(int dt, const Plan& pl, const Params& p) {
  const bool one_block = (pl.W == 1 && pl.NSUB == 1) ||
                         ((int64_t)pl.QPG * pl.LU <= 32) || (pl.ngroups == 1 && pl.nunits * pl.LU <= 32);
  return (dt == LIK_BF16 || dt == LIK_F16) && one_block && pl.dpad >= 64 && pl.dpad <= 512 &&
         ((uintptr_t)p.d.data) % 16 == 0 && p.d.sl_b % 16 == 0 && (p.d.cu || p.d.sn_b % 16 == 0) &&
         ((!p.amax && !(p.normalize & 2)) || pl.dpad == 128) && !p.pair_q && !p.pair_d && !p.d.mask && !p.d.ts &&
         !p.q.ts &&
         !p.scale_q && !p.scale_d && p.doc_filter != 2 && !p.accumulate &&
         (int64_t)q1_docs_per_wave(p) * pl.QPG <= kQ1Scores && p.forced_w <= 1;
}

int launch_q1(int dt, const Plan& pl, const Params& p0, hipStream_t s) {
  Params p = p0;
  // units of the group in one 32-column block (unit t keeps its place t, so
  // the column sums keep the tile kernel's order)
  if ((int64_t)p.QPG * p.LU > 32) p.QPG = 32 / p.LU;
  p.R = q1_docs_per_wave(p0);
  p.NR = (p.ndocs_pg + p.R - 1) / p.R;
  const bool normq = (p.normalize & 1) != 0;
  if (pl.dpad == 64)
    return dt == LIK_BF16 ? launch_q1_t<EK_BF16, 64>(p, normq, s) : launch_q1_t<EK_F16, 64>(p, normq, s);
  if (pl.dpad == 256)
    return dt == LIK_BF16 ? launch_q1_t<EK_BF16, 256>(p, normq, s) : launch_q1_t<EK_F16, 256>(p, normq, s);
  if (pl.dpad == 512)
    return dt == LIK_BF16 ? launch_q1_t<EK_BF16, 512>(p, normq, s) : launch_q1_t<EK_F16, 512>(p, normq, s);
  return dt == LIK_BF16 ? launch_q1_t<EK_BF16, 128>(p, normq, s) : launch_q1_t<EK_F16, 128>(p, normq, s);
}

}  // namespace lik
