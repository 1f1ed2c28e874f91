// Projection head fused into MaxSim for gfx950: scores of queries Q against
// docs given as hidden states H [Nd, Ld, d_model] and a linear head (W, b),
//   D[j, t] = normalize(H[j, t] @ W^T + b),  score[i, j] = sum_s max_t <Q[i, s], D[j, t]>,
// without forming D in memory. Semantics of the reference's fused head
// (late_interaction_kernels/fused_head.py:46-189, 262-332): fp32 projection of
// 16-bit H and W, bias and row L2-normalise in fp32, the normalised row
// rounded to the input dtype for the MaxSim product, a doc token that is
// masked (or past the doc's length) never wins, a query token whose doc has
// no valid token (or whose max is NaN or +inf) scores 0 and gets argmax -1,
// ties go to the lowest doc token.
//
// head_tile_kernel: one workgroup of 8 wavefronts per (doc j, chunk of 256
// doc tokens); wavefront w owns tokens [256 c + 32 w, +32).
//  * Projection as P^T = W . H^T on 32x32x16 MFMAs: W (A operand, 32 output
//    dims per lane row) is staged in LDS one k-unit (64 model dims) at a time,
//    double-buffered and shared by the 8 wavefronts; H (B operand, one doc
//    token per lane row) is read with coalesced, non-temporal buffer loads
//    (8 lanes x 16 bytes per 128-byte row segment) into registers three units
//    ahead of the MFMAs, and turned into B fragments through the wavefront's
//    LDS tile. Within a unit, lane half h supplies model dims [32 h, 32 h + 32)
//    and k-step kk the 8 dims at 8 kk of them: the same order for W and H, so
//    the contraction runs over the same dims whatever the pairing.
//  * The accumulators start at the bias. Element e of lane (l32, h) holds
//    output dim 32 n + 8 (e / 4) + 4 h + e % 4 of doc token l32, so a token's
//    squared norm is the lane's sum plus its partner lane's (l32 + 32).
//  * The normalised, rounded values are the A operand of the MaxSim MFMAs
//    as they sit: k-step (n, kk2) is the lane's elements 8 kk2 .. 8 kk2 + 7,
//    and the query fragments (B operand, staged once per workgroup in LDS)
//    are built with that same dim order. No transpose through LDS.
//  * Max over the 32 tokens in registers (plus one exchange between the lane
//    halves), then over the 8 wavefronts in LDS in token order; the chunk's
//    (max, argmax) per query token goes to the workspace.
// Calls with at most 64 query tokens (the inference case) run
// head_persist_kernel below instead (the same arithmetic and partial maxima;
// one persistent workgroup per CU streaming H and W into LDS by DMA), after
// head_valid_kernel has written the token-validity words it reads (with a
// doc mask or lengths; without, the persistent kernel computes them from the
// padded length).
// head_finish_kernel: per (query i, doc j), the chunks in order, then the sum
// over the query tokens in order: a fixed order, so the bits do not depend on
// scheduling.
#include "lik_common.h"

namespace lik {

namespace {

// 8 wavefronts per workgroup measured faster than 4 (two workgroups per CU)
constexpr int HEAD_WAVES = 8;
// cache policy of the H loads: 2 = non-temporal (each byte of H is read once)
constexpr int HEAD_H_AUX = 2;
constexpr int HEAD_THREADS = 64 * HEAD_WAVES;
constexpr int HEAD_ROWS = 32 * HEAD_WAVES;  // doc tokens per workgroup
constexpr int HEAD_MAXCOL = 256;            // query tokens (Nq * Lq) per call
constexpr int HEAD_MAXNB = 4;               // 32-wide output blocks (d_out <= 128)

struct HeadParams {
  const char* q;  // Q rows: q + i * q_sn + s * q_sl (bytes)
  int64_t q_sn, q_sl;
  const char* h;  // H rows: h + j * h_sn + t * h_sl (bytes)
  int64_t h_sn, h_sl;
  const char* w;  // W rows: w + o * w_sl (bytes)
  int64_t w_sl;
  const float* bias;       // [d_out] fp32, or null
  const uint16_t* bias16;  // [d_out] in the Q / H dtype (LIK_BIAS_16), or null
  const int8_t* dmask;  // keep flags, or null
  int64_t dm_sn, dm_sl;
  const int32_t* dlen;  // doc lengths, or null
  float2* part;         // [ncol][nd][nchunk] (max, argmax bits)
  float* out;
  int64_t os_q, os_d;
  int32_t* amax;  // [(i * nd + j) * lq + s], or null
  int nq, lq, ncol, nd, ld, dmodel, dout, nchunk, nunit, norm;
};

constexpr uint32_t kHeadOOB = 0xffffffffu;  // buffer offset past num_records: the load returns 0, no fetch

__device__ __forceinline__ __amdgpu_buffer_rsrc_t head_rsrc(const void* base, uint32_t nbytes) {
  // dword3 0x00020000: raw (untyped) access, stride 0, byte range check
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)nbytes, 0x00020000);
}

// output dim o's bias as fp32 (0 past d_out or without a bias)
template <int EK>
__device__ __forceinline__ float head_bias(const HeadParams& p, int o) {
  if (o >= p.dout) return 0.f;
  if (p.bias) return p.bias[o];
  if (p.bias16) return EK == EK_F16 ? f16_to_f32(p.bias16[o]) : bf16lo_to_f32(p.bias16[o]);
  return 0.f;
}

template <int EK>
__device__ __forceinline__ uint32_t to16(float f) {
  if constexpr (EK == EK_F16) return f32_to_f16_bits(f);
  else return f32_to_bf16_bits(f);
}

template <int EK>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return to16<EK>(a) | (to16<EK>(b) << 16);
}

template <int EK, int NB>
__global__ void __launch_bounds__(HEAD_THREADS) head_tile_kernel(const HeadParams p) {
  constexpr int KS2 = 2 * NB;  // MaxSim k-steps over the (padded) output dims
  __shared__ u32x4 s_w[2][NB * 4 * 64];
  extern __shared__ u32x4 s_q[];  // [ncb * KS2 * 64], sized at launch
  __shared__ float2 s_red[HEAD_WAVES][HEAD_MAXCOL];
  __shared__ float s_bias[32 * NB];
  __shared__ u32x4 s_h[HEAD_WAVES * 32 * 9];  // per-wave H unit tile

  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t j = blockIdx.x / p.nchunk;
  const int chunk = blockIdx.x - (int)j * p.nchunk;
  const int ncb = (p.ncol + 31) >> 5;

  // query fragments: k-step ks = (n, kk2) of column block cb, lane (col, h):
  // dims 32 n + 16 kk2 + 4 h + {0..3} and the same + 8
  for (int f = tid; f < ncb * KS2 * 64; f += HEAD_THREADS) {
    const int ln = f & 63, ks = (f >> 6) % KS2, cb = f / (64 * KS2);
    const int col = cb * 32 + (ln & 31), h = ln >> 5;
    const int base = 32 * (ks >> 1) + 16 * (ks & 1) + 4 * h;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (col < p.ncol) {
      const int i = col / p.lq, s = col - i * p.lq;
      const uint16_t* row = (const uint16_t*)(p.q + i * p.q_sn + s * p.q_sl);
      uint32_t e16[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int d = base + (k < 4 ? k : k + 4);
        e16[k] = d < p.dout ? row[d] : 0u;
      }
      v = u32x4{e16[0] | (e16[1] << 16), e16[2] | (e16[3] << 16), e16[4] | (e16[5] << 16), e16[6] | (e16[7] << 16)};
    }
    s_q[f] = v;
  }
  if (tid < 32 * NB) s_bias[tid] = head_bias<EK>(p, tid);

  // this lane's doc token and whether it takes part (in the doc, kept)
  const int t = chunk * HEAD_ROWS + wave * 32 + l32;
  const int dl = p.dlen ? min(p.dlen[j], p.ld) : p.ld;
  bool valid = t < dl;
  if (valid && p.dmask) valid = p.dmask[j * p.dm_sn + (int64_t)t * p.dm_sl] != 0;
  const uint64_t vb = __ballot(valid);
  const bool wave_on = (uint32_t)vb != 0u;  // any kept token in this wave's 32
  // Every global load of the loop is issued by every lane (an offset out of
  // range returns 0 without a fetch), so the compiler can count them.
  // H: this doc's rows [0, ld); a lane whose token is not kept fetches nothing
  const __amdgpu_buffer_rsrc_t rh =
      head_rsrc(p.h + j * p.h_sn, (uint32_t)((int64_t)(p.ld - 1) * p.h_sl + 2 * (int64_t)p.dmodel));
  // W fragment f = (n, kk, lane) of unit u: out dim 32 n + l32, model dims
  // 64 u + 32 h + 8 kk .. + 8
  const __amdgpu_buffer_rsrc_t rw =
      head_rsrc(p.w, (uint32_t)((int64_t)(p.dout - 1) * p.w_sl + 2 * (int64_t)p.dmodel));
  // fragments per thread: the unit has NB * 256 of them
  constexpr int WPT = (NB * 256 + HEAD_THREADS - 1) / HEAD_THREADS;
  auto load_w = [&](u32x4* dst, int u) {
#pragma unroll
    for (int k = 0; k < WPT; ++k) {
      const int f = tid + HEAD_THREADS * k;
      const int o = 32 * (f >> 8) + (f & 31), hw = (f >> 5) & 1, kw = (f >> 6) & 3;
      const int e = 64 * u + 32 * hw + 8 * kw;
      const bool on = f < NB * 256 && o < p.dout && e < p.dmodel;
      dst[k] = __builtin_amdgcn_raw_buffer_load_b128(rw, on ? (uint32_t)(o * p.w_sl) + 2u * (uint32_t)e : kHeadOOB, 0, 0);
    }
  };
  auto store_w = [&](int buf, const u32x4* v) {
#pragma unroll
    for (int k = 0; k < WPT; ++k)
      if (tid + HEAD_THREADS * k < NB * 256) s_w[buf][tid + HEAD_THREADS * k] = v[k];
  };
  // H unit u of this wave's 32 tokens: instruction c reads tokens 8 c .. 8 c + 7,
  // 8 lanes x 16 bytes each (coalesced 128-byte row segments); a token that is
  // not kept fetches nothing. The unit goes through the wave's LDS tile
  // (rows padded to 144 bytes: conflict-free fragment reads) into the B
  // fragments: lane (l32, h), k-step kk = token l32, model dims 64 u + 32 h + 8 kk.
  const int crow = lane >> 3, cseg = lane & 7;
  uint32_t coff[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int r = 8 * c + crow;
    coff[c] = ((vb >> r) & 1u) ? (uint32_t)((int64_t)(chunk * HEAD_ROWS + wave * 32 + r) * p.h_sl) + 16u * cseg
                               : kHeadOOB;
  }
  // (a unit past the row's end, u >= nunit included, is out of range by the
  // byte test alone: offsets are selected, never branched around)
  const uint32_t row_bytes = 2u * (uint32_t)p.dmodel;
  auto load_h = [&](u32x4* dst, int u) {
    const uint32_t ub = 128u * (uint32_t)u;
    const bool inrow = ub + 16u * cseg < row_bytes;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      dst[c] = __builtin_amdgcn_raw_buffer_load_b128(rh, (inrow && coff[c] != kHeadOOB) ? coff[c] + ub : kHeadOOB, 0,
                                                     HEAD_H_AUX);
  };
  u32x4* tile = s_h + wave * (32 * 9);  // 32 rows x 9 slots of 16 bytes
  auto frag_h = [&](const u32x4* g, u32x4* bf) {
#pragma unroll
    for (int c = 0; c < 4; ++c) tile[(8 * c + crow) * 9 + cseg] = g[c];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) bf[kk] = tile[l32 * 9 + 4 * hh + kk];
  };

  // accumulators start at the bias
  f32x16 acc[NB];
  __syncthreads();  // s_bias
#pragma unroll
  for (int n = 0; n < NB; ++n) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[n][4 * g + r] = s_bias[32 * n + 8 * g + 4 * hh + r];
    }
  }
  // H and W three units ahead of the MFMAs (register rings of 4; W unit u + 1
  // goes to LDS at the end of step u)
  u32x4 hb[4][4];
  u32x4 wr[4][WPT];
  load_w(wr[0], 0);
  store_w(0, wr[0]);
  load_w(wr[1], 1);
  load_w(wr[2], 2);
  load_h(hb[0], 0);
  load_h(hb[1], 1);
  load_h(hb[2], 2);
  __syncthreads();

  auto step = [&](auto slot_c, int u) {
    constexpr int S = decltype(slot_c)::value;  // u % 4
    load_w(wr[(S + 3) & 3], u + 3);  // past the last unit: out of range, no fetch
    load_h(hb[(S + 3) & 3], u + 3);
    u32x4 bf[4];
    frag_h(hb[S], bf);
    const u32x4* sw = s_w[u & 1];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
      for (int n = 0; n < NB; ++n) {
        const u32x4 a = sw[(n * 4 + kk) * 64 + lane];
        acc[n] = mfma32<EK>(acc[n], &a, &bf[kk]);
      }
    }
    store_w((u + 1) & 1, wr[(S + 1) & 3]);
    __syncthreads();
  };
  // A straight-line body (no branches for the compiler's load counting to
  // merge): the unit count is rounded up to a multiple of 4, the extra steps
  // load nothing (out of range: zeros) and add 0.
  for (int u = 0; u < p.nunit; u += 4) {
    step(std::integral_constant<int, 0>{}, u);
    step(std::integral_constant<int, 1>{}, u + 1);
    step(std::integral_constant<int, 2>{}, u + 2);
    step(std::integral_constant<int, 3>{}, u + 3);
  }

  // row L2 normalise (x / max(||x||, 1e-12)), round to the input dtype: the
  // A fragments of the MaxSim MFMAs
  float ss = 0.f;
#pragma unroll
  for (int n = 0; n < NB; ++n)
#pragma unroll
    for (int e = 0; e < 16; ++e) ss = fmaf(acc[n][e], acc[n][e], ss);
  ss += __shfl_xor(ss, 32);
  const float inv = p.norm ? inv_norm(ss) : 1.f;
  u32x4 df[KS2];
#pragma unroll
  for (int n = 0; n < NB; ++n) {
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const int e0 = 8 * k2;
      df[2 * n + k2] = u32x4{pack2<EK>(acc[n][e0] * inv, acc[n][e0 + 1] * inv),
                             pack2<EK>(acc[n][e0 + 2] * inv, acc[n][e0 + 3] * inv),
                             pack2<EK>(acc[n][e0 + 4] * inv, acc[n][e0 + 5] * inv),
                             pack2<EK>(acc[n][e0 + 6] * inv, acc[n][e0 + 7] * inv)};
    }
  }

  const uint32_t vrow = (uint32_t)vb;  // bit r: token r of this wave is kept
  for (int cb = 0; cb < ncb; ++cb) {
    float m = -INFINITY;
    int idx = -1;
    if (wave_on) {
      f32x16 c = {};
#pragma unroll
      for (int ks = 0; ks < KS2; ++ks) {
        const u32x4 b = s_q[(cb * KS2 + ks) * 64 + lane];
        c = mfma32<EK>(c, &df[ks], &b);
      }
      // element e: doc token 8 (e / 4) + 4 h + e % 4 (increasing in e), query column l32
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int r = 8 * (e >> 2) + 4 * hh + (e & 3);
        if ((vrow >> r) & 1u) {
          // a NaN similarity makes the max NaN (the token then scores 0)
          if (c[e] > m) idx = r;
          m = max_nan(m, c[e]);
        }
      }
      const float om = __shfl_xor(m, 32);
      const int oi = __shfl_xor(idx, 32);
      if (om > m || (om == m && oi >= 0 && (idx < 0 || oi < idx))) idx = oi;
      m = max_nan(m, om);
    }
    if (hh == 0) s_red[wave][cb * 32 + l32] = float2{m, __int_as_float(idx < 0 ? -1 : wave * 32 + idx)};
  }
  __syncthreads();
  if (tid < p.ncol) {
    float m = -INFINITY;
    int idx = -1;
    for (int w = 0; w < HEAD_WAVES; ++w) {
      const float2 v = s_red[w][tid];
      if (v.x > m) idx = __float_as_int(v.y);
      m = max_nan(m, v.x);
    }
    p.part[((int64_t)tid * p.nd + j) * p.nchunk + chunk] =
        float2{m, __int_as_float(idx < 0 ? -1 : chunk * HEAD_ROWS + idx)};
  }
}

// head_valid_kernel: one 32-bit word per (item, 32-token group) of the
// workgroup items (item = (doc j, chunk c); group g = tokens c * 256 + 32 g +
// 0..31): bit l set when that token is in the doc and kept. One wavefront per
// 64 tokens.
__global__ void __launch_bounds__(256) head_valid_kernel(const HeadParams p, uint32_t* __restrict__ words, int64_t nitems) {
  const int lane = threadIdx.x & 63;
  const int64_t gw = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (item, quarter)
  if (gw >= nitems * 4) return;
  const int64_t it = gw >> 2;
  const int64_t j = it / p.nchunk;
  const int c = (int)(it - j * p.nchunk);
  const int t = c * HEAD_ROWS + (int)(gw & 3) * 64 + lane;
  const int dl = p.dlen ? min(p.dlen[j], p.ld) : p.ld;
  bool valid = t < dl;
  if (valid && p.dmask) valid = p.dmask[j * p.dm_sn + (int64_t)t * p.dm_sl] != 0;
  const uint64_t b = __ballot(valid);
  if (lane == 0) {
    words[gw * 2] = (uint32_t)b;
    words[gw * 2 + 1] = (uint32_t)(b >> 32);
  }
}

// head_persist_kernel: the fused head for up to 64 query tokens, one
// persistent workgroup of 4 wavefronts per CU walking the (doc, chunk) items
// blockIdx.x, + gridDim.x, ... (a workgroup per item spent ~10 us per item
// filling and draining its load pipeline; here the pipeline runs on across
// items, and the query fragments are staged once). Wavefront w owns the item's
// tokens [64 w, 64 w + 64) as two 32-token groups that share every W fragment
// read. Per 64-dim unit:
//  * H through a ring of 3 unit tiles per wavefront (64 rows x 128 bytes),
//    unit u + 2 issued while unit u is multiplied (it may belong to the next
//    item): buffer_load ... lds, DMA instruction c writing rows 8 c .. 8 c + 7
//    (8 lanes x 16 bytes per row, a coalesced 128-byte segment); chunk k of
//    row r lands at slot 8 r + (k ^ ((r >> 1) & 7)), so a fragment read (32
//    rows, one chunk each) touches every bank group once per 16 lanes.
//  * W through two unit buffers shared by the wavefronts, unit u + 1 issued at
//    step u, NB blocks of 8 out dims x 128 bytes per wavefront (coalesced, the
//    same slot order as H).
//  * One wait per step: every wavefront issues NB + 8 DMA instructions per step
//    and loads complete in order, so `s_waitcnt vmcnt(8)` leaves exactly
//    H(u + 1) in flight; then one barrier (every wavefront's part of W(u) has
//    landed, every wavefront is done with what step u refills). The partial
//    maxima of a finished item are stored at the next step, before its wait
//    (one more instruction in flight: vmcnt(9) in the wavefront that stores).
//  * Token validity comes from head_valid_kernel's words by scalar loads, so
//    no vector load but the DMA runs in the loop (the compiler would wait for
//    all of them before using one).
constexpr int HP_WAVES = 4;
constexpr int HP_THREADS = 64 * HP_WAVES;
constexpr int HP_MAXCOL = 64;  // query tokens of the persistent kernel
static_assert(HP_WAVES * 64 == HEAD_ROWS, "doc tokens per item (the chunk layout of the partial maxima)");

// scalar load of two uniform words (read-only data; the scalar cache is only
// read). The load and its wait sit in one asm statement: a value the
// compiler sees as an asm output may be copied right after the asm.
__device__ __forceinline__ uint64_t sload_u64(const uint32_t* base, int64_t idx) {
  const uint64_t a = (uint64_t)(base + idx);
  uint64_t v;
  asm volatile("s_load_dwordx2 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=&s"(v) : "s"(a) : "memory");
  return v;
}

template <int EK, int NB>
__global__ void __launch_bounds__(HP_THREADS) head_persist_kernel(const HeadParams p, const uint32_t* __restrict__ vwords,
                                                                  int nitems) {
  constexpr int KS2 = 2 * NB;
  constexpr int WI = NB;  // W blocks (8 out dims each) per wavefront per unit
  constexpr float NEG_INF = -__builtin_huge_valf();
  __shared__ __attribute__((aligned(16))) char s_ring[HP_WAVES][3][64 * 128];
  __shared__ __attribute__((aligned(16))) u32x4 s_w[2][NB * 4 * 64];
  __shared__ __attribute__((aligned(16))) u32x4 s_q[(HP_MAXCOL / 32) * KS2 * 64];
  __shared__ float2 s_red[2 * HP_WAVES][HP_MAXCOL];
  __shared__ float s_bias[32 * NB];
  __shared__ uint32_t s_vw[4][HP_WAVES][2];  // validity words of item k (slot k % 4), per wavefront

  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ncb = (p.ncol + 31) >> 5;

  // query fragments (once): k-step ks = (n, kk2) of column block cb, lane
  // (col, h): dims 32 n + 16 kk2 + 4 h + {0..3} and the same + 8
  for (int f = tid; f < ncb * KS2 * 64; f += HP_THREADS) {
    const int ln = f & 63, ks = (f >> 6) % KS2, cb = f / (64 * KS2);
    const int col = cb * 32 + (ln & 31), h = ln >> 5;
    const int base = 32 * (ks >> 1) + 16 * (ks & 1) + 4 * h;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (col < p.ncol) {
      const int i = col / p.lq, sq = col - i * p.lq;
      const uint16_t* row = (const uint16_t*)(p.q + i * p.q_sn + sq * p.q_sl);
      uint32_t e16[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = base + (e < 4 ? e : e + 4);
        e16[e] = d < p.dout ? row[d] : 0u;
      }
      v = u32x4{e16[0] | (e16[1] << 16), e16[2] | (e16[3] << 16), e16[4] | (e16[5] << 16), e16[6] | (e16[7] << 16)};
    }
    s_q[f] = v;
  }
  if (tid < 32 * NB) s_bias[tid] = head_bias<EK>(p, tid);

  auto desc = [](const void* base, uint32_t nbytes) -> u32x4 {
    const uint64_t b = (uint64_t)base;
    return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b),
                 (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32) & 0xffffu),
                 (uint32_t)__builtin_amdgcn_readfirstlane(nbytes), 0x00020000u};
  };
  const u32x4 dw = desc(p.w, (uint32_t)((int64_t)(p.dout - 1) * p.w_sl + 2 * (int64_t)p.dmodel));
  const uint32_t hrec = (uint32_t)((int64_t)(p.ld - 1) * p.h_sl + 2 * (int64_t)p.dmodel);
  const uint32_t row_bytes = 2u * (uint32_t)p.dmodel;
  // W lane offsets (unit 0): block q = wave * WI + i holds out dims 8 q .. 8 q + 7;
  // lane chunk c of row o is model dims 8 c .. 8 c + 7 of the unit and lands
  // at slot 8 o + (c ^ ((o >> 1) & 7))
  uint32_t woff[WI], wdim[WI];
#pragma unroll
  for (int i = 0; i < WI; ++i) {
    const int q = wave * WI + i;
    const int o = 8 * q + (lane >> 3);
    const int c = (lane & 7) ^ ((o >> 1) & 7);
    wdim[i] = (uint32_t)(8 * c);
    woff[i] = o < p.dout ? (uint32_t)(o * p.w_sl) + 2u * wdim[i] : kHeadOOB;
  }
  // H lane constants: instruction c, row 8 c + lane / 8, its chunk's byte offset
  uint32_t hseg[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int r = 8 * c + (lane >> 3);
    hseg[c] = 16u * (uint32_t)((lane & 7) ^ ((r >> 1) & 7));
  }
  auto lds_addr = [](const void* ptr) -> uint32_t {
    return (uint32_t)__builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const char*)ptr);
  };
  const uint32_t ring0 = lds_addr(&s_ring[wave][0][0]);
  const uint32_t w0 = lds_addr(&s_w[0][wave * WI * 64]);
  auto dma = [](uint32_t lds, uint32_t voff, const u32x4& dsc, auto NT) {
    uint32_t saved;
    if constexpr (decltype(NT)::value)
      asm volatile(
          "s_mov_b32 %0, m0\n\t"
          "s_mov_b32 m0, %1\n\t"
          "s_nop 0\n\t"  // an M0 write needs one wait state before an LDS DMA reads it
          "buffer_load_dwordx4 %2, %3, 0 offen nt lds\n\t"
          "s_mov_b32 m0, %0"
          : "=&s"(saved)
          : "s"(lds), "v"(voff), "s"(dsc)
          : "memory");
    else
      asm volatile(
          "s_mov_b32 %0, m0\n\t"
          "s_mov_b32 m0, %1\n\t"
          "s_nop 0\n\t"
          "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
          "s_mov_b32 m0, %0"
          : "=&s"(saved)
          : "s"(lds), "v"(voff), "s"(dsc)
          : "memory");
  };

  const int G = gridDim.x, b0 = blockIdx.x;
  const int nk = (nitems - b0 + G - 1) / G;  // items of this workgroup (b0 < nitems)
  const int nunit = p.nunit;

  // ---- H issue cursor: item hk of this workgroup, unit hu; lane offsets of
  // the item's rows (kOOB: token not kept, or no item) and its descriptor ----
  // Every step starts by loading (scalar) the words of the item after the
  // cursor's, under the same wait as the step's DMA, so the cursor has them
  // when it enters that item; the item's words also go to s_vw for its
  // epilogue.
  int hk = 0, hu = 0;
  uint32_t hoff[8];
  u32x4 dh;
  uint64_t wnext = 0;
  auto set_h_item = [&](int k) {
    if (k < nk) {
      const int it = b0 + k * G;
      const int64_t j = it / p.nchunk;
      const int chunk = it - (int)j * p.nchunk;
      const uint32_t v0 = (uint32_t)wnext, v1 = (uint32_t)(wnext >> 32);
      if (lane == 0) {
        s_vw[k & 3][wave][0] = v0;
        s_vw[k & 3][wave][1] = v1;
      }
      dh = desc(p.h + j * p.h_sn, hrec);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int r = 8 * c + (lane >> 3);
        const uint32_t vw = c < 4 ? v0 : v1;
        hoff[c] = ((vw >> (r & 31)) & 1u) ? (uint32_t)((int64_t)(chunk * HEAD_ROWS + wave * 64 + r) * p.h_sl) + hseg[c]
                                          : kHeadOOB;
      }
    } else {
#pragma unroll
      for (int c = 0; c < 8; ++c) hoff[c] = kHeadOOB;
    }
  };
  // H(U) for the cursor's unit into ring stage U % 3, then advance the cursor
  // (wnext: the words of item hk + 1)
  auto issue_h = [&](int U) {
    const uint32_t ub = 128u * (uint32_t)hu;
    const uint32_t st = ring0 + (uint32_t)((U % 3) * 64 * 128);
#pragma unroll
    for (int c = 0; c < 8; ++c)
      dma(st + (uint32_t)(c * 1024), (hoff[c] != kHeadOOB && ub + hseg[c] < row_bytes) ? hoff[c] + ub : kHeadOOB, dh,
          std::true_type{});
    if (++hu == nunit) {
      hu = 0;
      set_h_item(++hk);
    }
  };
  // W(U): unit U % nunit into buffer U % 2
  auto issue_w = [&](int U) {
    const int u = U % nunit;
    const uint32_t ub = 128u * (uint32_t)u;
#pragma unroll
    for (int i = 0; i < WI; ++i)
      dma(w0 + (uint32_t)((U & 1) * NB * 4 * 64 * 16 + i * 1024),
          (woff[i] != kHeadOOB && 64u * u + wdim[i] < (uint32_t)p.dmodel) ? woff[i] + ub : kHeadOOB, dw,
          std::false_type{});
  };

  f32x16 acc[2][NB];
  auto reset_acc = [&]() {
#pragma unroll
    for (int n = 0; n < NB; ++n) {
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[0][n][e] = s_bias[32 * n + 8 * (e >> 2) + 4 * hh + (e & 3)];
      acc[1][n] = acc[0][n];
    }
  };
  __syncthreads();  // s_q, s_bias
  reset_acc();
  // Validity words of this wavefront's 64 tokens of item k (item 0 past the
  // last): loaded from head_valid_kernel's output, or, with no mask and no
  // lengths (vwords null: every token before the doc's end is kept),
  // computed from the padded length alone.
  const bool has_words = vwords != nullptr;
  auto words_addr = [&](int k) -> const uint32_t* {
    return vwords + (int64_t)(b0 + (k < nk ? k : 0) * G) * 8 + wave * 2;
  };
  auto words_of = [&](int k) -> uint64_t {
    const int it = b0 + (k < nk ? k : 0) * G;
    const int chunk = it - (it / p.nchunk) * p.nchunk;
    const int n = p.ld - (chunk * HEAD_ROWS + wave * 64);  // tokens of the 64 inside the doc
    return n >= 64 ? ~0ull : (n <= 0 ? 0ull : (1ull << n) - 1ull);
  };
  auto words = [&](int k) -> uint64_t { return has_words ? sload_u64(words_addr(k), 0) : words_of(k); };
  wnext = words(0);
  set_h_item(0);
  wnext = words(hk + 1);
  issue_h(0);
  issue_w(0);
  wnext = words(hk + 1);
  issue_h(1);
  // this lane's fragment chunk offsets within 32 rows (row l32, chunk 4 h + kk;
  // (row >> 1) & 7 is (l32 >> 1) & 7 for every 32-row group), for H and W alike
  uint32_t fo[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) fo[kk] = (uint32_t)(l32 * 8 + ((4 * hh + kk) ^ ((l32 >> 1) & 7))) * 16u;

  const bool stores = wave * 64 < p.ncol;  // this wavefront writes partial maxima
  bool pend = false;                       // an item's partial maxima wait to be stored
  float2 pval = {0.f, 0.f};
  float2* pdst = nullptr;
  int k = 0, u = 0;
  const int NU = nk * nunit;
  for (int U = 0; U < NU; ++U) {
    if (has_words) {
      const uint64_t wa = (uint64_t)words_addr(hk + 1);
      if (pend && stores) {
        if (tid < p.ncol) *pdst = pval;
        asm volatile("s_load_dwordx2 %0, %1, 0x0\n\ts_waitcnt vmcnt(9) lgkmcnt(0)\n\ts_barrier"
                     : "=&s"(wnext) : "s"(wa) : "memory");
      } else {
        asm volatile("s_load_dwordx2 %0, %1, 0x0\n\ts_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier"
                     : "=&s"(wnext) : "s"(wa) : "memory");
      }
    } else {
      if (pend && stores) {
        if (tid < p.ncol) *pdst = pval;
        asm volatile("s_waitcnt vmcnt(9) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      }
      wnext = words_of(hk + 1);
    }
    pend = false;
    issue_w(U + 1);
    issue_h(U + 2);
    const char* st = &s_ring[wave][U % 3][0];
    const char* sw = (const char*)s_w[U & 1];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const u32x4 b0v = *(const u32x4*)(st + fo[kk]);
      const u32x4 b1v = *(const u32x4*)(st + 32 * 128 + fo[kk]);
#pragma unroll
      for (int n = 0; n < NB; ++n) {
        const u32x4 a = *(const u32x4*)(sw + n * 256 * 16 + fo[kk]);
        acc[0][n] = mfma32<EK>(acc[0][n], &a, &b0v);
        acc[1][n] = mfma32<EK>(acc[1][n], &a, &b1v);
      }
    }
    if (++u < nunit) continue;
    // ---- item k done: normalise, MaxSim against the query block, maxima over
    // the item's 8 token groups in token order ----
    u = 0;
    // One wavefront runs per SIMD, so the epilogue is written for
    // instruction-level parallelism: both groups side by side, squared norms
    // in four partial sums, the MaxSim product as four independent MFMA
    // chains (even / odd k-steps of each group, added at the end) on query
    // fragments loaded up front, and the masked max / argmax over the two
    // halves of the elements, merged in index order (a later half wins only
    // when strictly larger, as in one scan).
    const int it = b0 + k * G;
    const int64_t j = it / p.nchunk;
    const int chunk = it - (int)j * p.nchunk;
    uint32_t vrow[2];
    u32x4 df[2][KS2];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      vrow[g] = __builtin_amdgcn_readfirstlane(s_vw[k & 3][wave][g]);  // bit r: token r of the group is kept
      float s4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int n = 0; n < NB; ++n)
#pragma unroll
        for (int e = 0; e < 16; ++e) s4[e & 3] = fmaf(acc[g][n][e], acc[g][n][e], s4[e & 3]);
      float ss = (s4[0] + s4[1]) + (s4[2] + s4[3]);
      ss += __shfl_xor(ss, 32);
      const float inv = p.norm ? inv_norm(ss) : 1.f;
#pragma unroll
      for (int n = 0; n < NB; ++n) {
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
          const int e0 = 8 * k2;
          df[g][2 * n + k2] = u32x4{pack2<EK>(acc[g][n][e0] * inv, acc[g][n][e0 + 1] * inv),
                                    pack2<EK>(acc[g][n][e0 + 2] * inv, acc[g][n][e0 + 3] * inv),
                                    pack2<EK>(acc[g][n][e0 + 4] * inv, acc[g][n][e0 + 5] * inv),
                                    pack2<EK>(acc[g][n][e0 + 6] * inv, acc[g][n][e0 + 7] * inv)};
        }
      }
    }
    for (int cb = 0; cb < ncb; ++cb) {
      u32x4 qb[KS2];
#pragma unroll
      for (int ks = 0; ks < KS2; ++ks) qb[ks] = s_q[(cb * KS2 + ks) * 64 + lane];
      f32x16 c0[2] = {{}, {}}, c1[2] = {{}, {}};
#pragma unroll
      for (int ks = 0; ks < KS2; ks += 2) {
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          c0[g] = mfma32<EK>(c0[g], &df[g][ks], &qb[ks]);
          c1[g] = mfma32<EK>(c1[g], &df[g][ks + 1], &qb[ks + 1]);
        }
      }
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const f32x16 c = c0[g] + c1[g];
        // element e: doc token 8 (e / 4) + 4 h + e % 4 (increasing in e), query column l32
        float mh[2] = {NEG_INF, NEG_INF};
        int ih[2] = {-1, -1};
        const uint32_t vh = vrow[g] >> (4 * hh);  // bit 8 j + i: element 4 j + i is a kept token
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = 8 * (e >> 2) + 4 * hh + (e & 3);
          // selects, not branches: a dropped token is -inf and never the argmax;
          // a NaN similarity makes the max NaN (the token then scores 0)
          const float x = ((vh >> (8 * (e >> 2) + (e & 3))) & 1u) ? c[e] : NEG_INF;
          ih[e >> 3] = x > mh[e >> 3] ? r : ih[e >> 3];
          mh[e >> 3] = max_nan(mh[e >> 3], x);
        }
        int idx = mh[1] > mh[0] ? ih[1] : ih[0];
        float m = max_nan(mh[0], mh[1]);
        const float om = __shfl_xor(m, 32);
        const int oi = __shfl_xor(idx, 32);
        if (om > m || (om == m && oi >= 0 && (idx < 0 || oi < idx))) idx = oi;
        m = max_nan(m, om);
        const int grp = wave * 2 + g;  // 32-token group of the item, in token order
        if (hh == 0) s_red[grp][cb * 32 + l32] = float2{m, __int_as_float(idx < 0 ? -1 : grp * 32 + idx)};
      }
    }
    // (LDS only: __syncthreads would also wait for every DMA in flight)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (tid < p.ncol) {
      float m = NEG_INF;
      int idx = -1;
#pragma unroll
      for (int w = 0; w < 2 * HP_WAVES; ++w) {
        const float2 v = s_red[w][tid];
        if (v.x > m) idx = __float_as_int(v.y);
        m = max_nan(m, v.x);
      }
      pval = float2{m, __int_as_float(idx < 0 ? -1 : chunk * HEAD_ROWS + idx)};
      pdst = &p.part[((int64_t)tid * p.nd + j) * p.nchunk + chunk];
    }
    pend = true;
    ++k;
    reset_acc();
  }
  if (pend && stores && tid < p.ncol) *pdst = pval;
  // no DMA may still be writing this workgroup's LDS when it exits
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// One wavefront per (query i, doc j): lane l takes query tokens l, l + 64, ...
// (chunks in order, then its tokens in order), then a fixed shuffle tree.
__global__ void __launch_bounds__(256) head_finish_kernel(const HeadParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t u = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (u >= (int64_t)p.nq * p.nd) return;
  const int64_t i = u / p.nd, j = u - i * p.nd;
  float sum = 0.f;
  for (int s = lane; s < p.lq; s += 64) {
    const int64_t col = i * p.lq + s;
    float m = -INFINITY;
    int idx = -1;
    for (int c = 0; c < p.nchunk; ++c) {
      const float2 v = p.part[(col * p.nd + j) * p.nchunk + c];
      if (v.x > m) idx = __float_as_int(v.y);
      m = max_nan(m, v.x);
    }
    // no kept token (-inf) or a NaN / +inf max: the token scores 0, argmax -1
    const bool any = __builtin_isfinite(m);
    sum += any ? m : 0.f;
    if (p.amax) p.amax[(i * p.nd + j) * p.lq + s] = any ? idx : -1;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o);
  if (lane == 0) p.out[i * p.os_q + j * p.os_d] = sum;
}

template <int EK>
int launch_head(const HeadParams& p, uint32_t* vwords, hipStream_t s) {
  const int nb = (p.dout + 31) / 32;
  const int64_t grid = (int64_t)p.nd * p.nchunk;
  if (grid > 0) {
    // query fragments: 32-column blocks x 2 NB k-steps x 64 lanes x 16 bytes
    const size_t qlds = (size_t)((p.ncol + 31) / 32) * (2 * nb) * 64 * 16;
    const dim3 g((unsigned)grid), b(HEAD_THREADS);
    if (p.ncol <= HP_MAXCOL) {
      // token-validity words, then one persistent workgroup per CU
      const int64_t nitems = grid;
      if (nitems > 0x7fffffffLL) return LIK_ERR_UNSUPPORTED;
      // without a mask or lengths every token before the doc's end is kept:
      // the persistent kernel computes those words itself
      if (p.dmask || p.dlen) {
        hipLaunchKernelGGL(head_valid_kernel, dim3((unsigned)((nitems * 4 + 3) / 4)), dim3(256), 0, s, p, vwords,
                           nitems);
        if (hipGetLastError() != hipSuccess) return LIK_ERR_LAUNCH;
      } else {
        vwords = nullptr;
      }
      int dev = 0, ncu = 0;
      if (hipGetDevice(&dev) != hipSuccess ||
          hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu < 1)
        return LIK_ERR_LAUNCH;
      const int pg = (int)(nitems < ncu ? nitems : ncu);
      const dim3 gp((unsigned)pg), bp(HP_THREADS);
      auto go = [&](auto kern) { hipLaunchKernelGGL(kern, gp, bp, 0, s, p, vwords, (int)nitems); };
      switch (nb) {
        case 1: go(head_persist_kernel<EK, 1>); break;
        case 2: go(head_persist_kernel<EK, 2>); break;
        case 3: go(head_persist_kernel<EK, 3>); break;
        default: go(head_persist_kernel<EK, 4>); break;
      }
    } else {
      switch (nb) {
        case 1: hipLaunchKernelGGL((head_tile_kernel<EK, 1>), g, b, qlds, s, p); break;
        case 2: hipLaunchKernelGGL((head_tile_kernel<EK, 2>), g, b, qlds, s, p); break;
        case 3: hipLaunchKernelGGL((head_tile_kernel<EK, 3>), g, b, qlds, s, p); break;
        default: hipLaunchKernelGGL((head_tile_kernel<EK, 4>), g, b, qlds, s, p); break;
      }
    }
    if (hipGetLastError() != hipSuccess) return LIK_ERR_LAUNCH;
  }
  const int64_t nu = (int64_t)p.nq * p.nd;
  hipLaunchKernelGGL(head_finish_kernel, dim3((unsigned)((nu + 3) / 4)), dim3(256), 0, s, p);
  return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
}

// shape checks shared by the entry point and its workspace query
int head_check(const lik_seqs_t* Q, const lik_seqs_t* H, const void* W, int64_t w_stride) {
  if (!Q || !H) return LIK_ERR_INVALID;
  if (Q->dtype != H->dtype) return LIK_ERR_INVALID;
  if (Q->dtype != LIK_BF16 && Q->dtype != LIK_F16) return LIK_ERR_UNSUPPORTED;
  if (Q->n < 0 || Q->len < 0 || H->n < 0 || H->len < 0 || Q->dim <= 0 || H->dim <= 0) return LIK_ERR_INVALID;
  if (Q->cu_seqlens || Q->lengths || Q->mask || Q->token_scale) return LIK_ERR_UNSUPPORTED;
  if (H->cu_seqlens || H->token_scale) return LIK_ERR_UNSUPPORTED;
  if (Q->dim > 32 * HEAD_MAXNB || Q->n * Q->len > HEAD_MAXCOL) return LIK_ERR_UNSUPPORTED;
  if (H->dim % 8 || H->stride_n % 8 || H->stride_l % 8 || w_stride % 8 || w_stride < H->dim) return LIK_ERR_UNSUPPORTED;
  if (H->len > 0x7fffff00LL || H->n > 0x7fffffffLL) return LIK_ERR_UNSUPPORTED;
  // 32-bit buffer offsets: one doc's rows and all of W within 4 GB
  if (H->len * H->stride_l * 2 >= ((int64_t)1 << 32) - 256 || Q->dim * w_stride * 2 >= ((int64_t)1 << 32) - 256)
    return LIK_ERR_UNSUPPORTED;
  if (((uintptr_t)H->data) % 16 || ((uintptr_t)W) % 16) return LIK_ERR_UNSUPPORTED;
  return LIK_OK;
}

size_t head_part_bytes(const lik_seqs_t* Q, const lik_seqs_t* H) {
  const int64_t nchunk = (H->len + HEAD_ROWS - 1) / HEAD_ROWS;
  return (size_t)(Q->n * Q->len) * (size_t)H->n * (size_t)nchunk * sizeof(float2);
}

// token-validity words of the persistent kernel: 8 per (doc, chunk)
size_t head_word_bytes(const lik_seqs_t* Q, const lik_seqs_t* H) {
  const int64_t nchunk = (H->len + HEAD_ROWS - 1) / HEAD_ROWS;
  return (Q->n * Q->len > 0 && Q->n * Q->len <= HP_MAXCOL) ? (size_t)H->n * (size_t)nchunk * 8 * sizeof(uint32_t) : 0;
}

}  // namespace

}  // namespace lik

using namespace lik;

extern "C" {

size_t lik_maxsim_from_hidden_workspace_size(const lik_seqs_t* Q, const lik_seqs_t* H) {
  if (!Q || !H || Q->n < 0 || Q->len < 0 || H->n < 0 || H->len < 0) return 0;
  const size_t b = head_part_bytes(Q, H), w = head_word_bytes(Q, H);
  return b ? ((b + 255) & ~(size_t)255) + w + 256 : 0;
}

int lik_maxsim_from_hidden(const lik_seqs_t* Q, const lik_seqs_t* H, const void* W, int64_t w_stride,
                           const void* bias, uint32_t flags, float* out, int64_t out_stride_q,
                           int64_t out_stride_d, int32_t* argmax, void* workspace, size_t workspace_bytes,
                           lik_stream_t stream) {
  int rc = head_check(Q, H, W, w_stride);
  if (rc != LIK_OK) return rc;
  if (flags & ~(uint32_t)(LIK_NORMALIZE_D | LIK_BIAS_16)) return LIK_ERR_INVALID;
  if (Q->n == 0 || H->n == 0) return LIK_OK;
  if (!out || !Q->data || (!H->data && H->len > 0) || !W) return LIK_ERR_INVALID;
  const size_t need = lik_maxsim_from_hidden_workspace_size(Q, H);
  if (need && (!workspace || workspace_bytes < need)) return LIK_ERR_WORKSPACE;
  HeadParams p{};
  p.q = (const char*)Q->data;
  p.q_sn = Q->stride_n * 2;
  p.q_sl = Q->stride_l * 2;
  p.h = (const char*)H->data;
  p.h_sn = H->stride_n * 2;
  p.h_sl = H->stride_l * 2;
  p.w = (const char*)W;
  p.w_sl = w_stride * 2;
  p.bias = (flags & LIK_BIAS_16) ? nullptr : (const float*)bias;
  p.bias16 = (flags & LIK_BIAS_16) ? (const uint16_t*)bias : nullptr;
  p.dmask = H->mask;
  p.dm_sn = H->mask_stride_n;
  p.dm_sl = H->mask_stride_l;
  p.dlen = H->lengths;
  p.part = (float2*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  p.out = out;
  p.os_q = out_stride_q;
  p.os_d = out_stride_d;
  p.amax = argmax;
  p.nq = (int)Q->n;
  p.lq = (int)Q->len;
  p.ncol = (int)(Q->n * Q->len);
  p.nd = (int)H->n;
  p.ld = (int)H->len;
  p.dmodel = H->dim;
  p.dout = Q->dim;
  p.nchunk = (int)((H->len + HEAD_ROWS - 1) / HEAD_ROWS);
  p.nunit = (H->dim + 63) / 64;
  p.norm = (flags & LIK_NORMALIZE_D) ? 1 : 0;
  if (p.lq == 0) {
    // no query tokens: every score is 0
    p.nchunk = 0;
  }
  uint32_t* vwords = (uint32_t*)((char*)p.part + ((head_part_bytes(Q, H) + 255) & ~(size_t)255));
  hipStream_t s = (hipStream_t)stream;
  return Q->dtype == LIK_F16 ? launch_head<EK_F16>(p, vwords, s) : launch_head<EK_BF16>(p, vwords, s);
}

}  // extern "C"
