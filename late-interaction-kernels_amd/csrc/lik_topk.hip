// Top-k selection and PLAID approximate scoring for gfx950.
//
// Top-k: each (score, index) candidate becomes one 64-bit key
//   key = order(score) << 32 | ~index
// where order() is the monotone float->uint32 map (descending scores map to
// descending keys; for largest=False the score part is complemented). Keys
// are unique and never 0 (indices stay below 2^32 - 1), and "larger key" ==
// "better score, then lower index", so the k best candidates are exactly the
// k largest keys and any grouping of the candidates selects the same set.
//
// One workgroup selects the kk largest of up to MAX_KEYS LDS-resident keys
// by an 8-pass MSB-first radix select (256-bin histograms), compacts the
// winners and bitonic-sorts them. A row wider than one workgroup's share is
// reduced as a tree: level 0 gives each MAX_N-score slice of a row its own
// workgroup, which writes its k best keys (0-padded) to a workspace; each
// further level merges up to MAX_KEYS / k such lists per workgroup, and the
// level with one group left writes scores and indices. The running list
// (prev_*) joins slice 0 at level 0.
// This replaces topk.py:41-86 / retrieve.py:278-305 (torch.topk + cat +
// gather per chunk) and pins the tie order torch.topk leaves unspecified.
#include "lik_common.h"

namespace lik {

constexpr int TK_THREADS = 256;
// Two LDS capacity classes. Small (k <= 1024): 4096 scores per level-0 group
// plus a running list, winners sorted in their own array (48 KB). Large
// (k <= 8192): 16384 keys (128 KB, one workgroup per CU), 8192 scores per
// level-0 group, winners compacted in place into the key array.
template <int CLS> struct TkCap;
template <> struct TkCap<0> {
  static constexpr int MAX_N = 4096, MAX_K = 1024, MAX_KEYS = MAX_N + MAX_K;
  static constexpr bool INPLACE = false;
};
template <> struct TkCap<1> {
  static constexpr int MAX_N = 8192, MAX_K = 8192, MAX_KEYS = MAX_N + MAX_K;
  static constexpr bool INPLACE = true;
};
constexpr int TK_MAX_N = TkCap<0>::MAX_N;
constexpr int TK_MAX_K = TkCap<1>::MAX_K;  // largest k of any class
inline int topk_class(int64_t k) { return k <= TkCap<0>::MAX_K ? 0 : 1; }

__device__ __forceinline__ uint32_t float_order(float f) {
  uint32_t b = __float_as_uint(f);
  if (b == 0x80000000u) b = 0u;  // -0 == +0
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float order_float(uint32_t o) {
  const uint32_t b = (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o;
  return __uint_as_float(b);
}
__device__ __forceinline__ uint64_t make_key(float s, uint32_t idx, int largest) {
  uint32_t o = float_order(s);
  if (!largest) o = ~o;
  return ((uint64_t)o << 32) | (uint64_t)(~idx);
}

struct TopkArgs {
  // level 0: scores [rows, n] (row stride ld), doc index = idx_base + column
  const float* scores;
  int64_t n, ld, idx_base;
  const float* prev_s;
  const int64_t* prev_i;
  int64_t pk, pld;
  // later levels: per row nin keys (lists of k) at keys_in + row * nin
  const uint64_t* keys_in;
  int64_t nin;
  int64_t k;
  int largest;
  int groups;        // groups per row at this level
  int64_t per_group; // scores (level 0) or keys (later levels) per group
  // output: keys_out + (row * groups + g) * k when groups > 1, else scores/indices
  uint64_t* keys_out;
  float* out_s;
  int64_t* out_i;
  int64_t old;
};

template <int CLS, bool FROM_KEYS>
__global__ void __launch_bounds__(TK_THREADS) topk_select_kernel(TopkArgs a) {
  using C = TkCap<CLS>;
  __shared__ uint64_t s_keys[C::MAX_KEYS];
  __shared__ uint64_t s_sel_own[C::INPLACE ? 1 : C::MAX_K];
  uint64_t* const s_sel = C::INPLACE ? s_keys : s_sel_own;
  __shared__ uint32_t s_hist[256];
  __shared__ uint64_t s_prefix, s_pmask;
  __shared__ int s_kk, s_done, s_cnt, s_real, s_fcnt;
  __shared__ int s_wcnt[TK_THREADS / 64];
  __shared__ uint64_t s_wmin[TK_THREADS / 64];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t row = blockIdx.x / a.groups;
  const int g = (int)(blockIdx.x - row * a.groups);
  if (tid == 0) s_real = 0;
  __syncthreads();

  int total;
  if (!FROM_KEYS && g == 0 && a.groups == 1 && a.pk > 0 && a.pk == a.k) {
    // A running merge whose list is full: every one of the k list keys is at
    // least the list's smallest key T, so a chunk key below T cannot be among
    // the k best of the union. Only chunk keys above T join the list's keys:
    // the same k winners, usually from ~k keys instead of k + n. (The list
    // need not be sorted; T is its minimum.)
    const int pk = (int)a.pk;
    uint64_t mn = ~0ull;
    for (int i = tid; i < pk; i += TK_THREADS) {
      const uint64_t key = make_key(a.prev_s[row * a.pld + i], (uint32_t)a.prev_i[row * a.pld + i], a.largest);
      s_keys[i] = key;
      mn = key < mn ? key : mn;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const uint64_t v = __shfl_xor(mn, o);
      mn = v < mn ? v : mn;
    }
    if (lane == 0) s_wmin[wv] = mn;
    if (tid == 0) s_fcnt = 0;
    __syncthreads();
    uint64_t T = s_wmin[0];
#pragma unroll
    for (int w = 1; w < TK_THREADS / 64; ++w) T = s_wmin[w] < T ? s_wmin[w] : T;
    const int nn = (int)min(a.per_group, a.n);
    for (int i0 = 0; i0 < nn; i0 += TK_THREADS) {
      const int i = i0 + tid;
      const uint64_t key = i < nn ? make_key(a.scores[row * a.ld + i], (uint32_t)(a.idx_base + i), a.largest) : 0;
      const bool win = i < nn && key > T;
      const uint64_t bal = __ballot(win);
      int base = 0;
      if (lane == 0 && bal) base = atomicAdd(&s_fcnt, (int)__popcll(bal));
      base = __shfl(base, 0);
      if (win) s_keys[pk + base + (int)__popcll(bal & ((1ull << lane) - 1ull))] = key;
    }
    __syncthreads();
    total = pk + s_fcnt;
    if (tid == 0) s_real = total;
  } else if (!FROM_KEYS) {
    const int64_t c0 = (int64_t)g * a.per_group;
    const int64_t nn = min(a.per_group, a.n - c0);
    const int pk = g == 0 ? (int)a.pk : 0;
    total = pk + (int)nn;
    for (int i = tid; i < total; i += TK_THREADS) {
      uint64_t key;
      if (i < pk) {
        key = make_key(a.prev_s[row * a.pld + i], (uint32_t)a.prev_i[row * a.pld + i], a.largest);
      } else {
        const int64_t c = c0 + (i - pk);
        key = make_key(a.scores[row * a.ld + c], (uint32_t)(a.idx_base + c), a.largest);
      }
      s_keys[i] = key;
    }
    if (tid == 0) s_real = total;
  } else {
    const int64_t c0 = (int64_t)g * a.per_group;
    total = (int)min(a.per_group, a.nin - c0);
    const uint64_t* src = a.keys_in + row * a.nin + c0;
    for (int i0 = 0; i0 < total; i0 += TK_THREADS) {
      const int i = i0 + tid;
      const uint64_t key = i < total ? src[i] : 0;
      if (i < total) s_keys[i] = key;
      const uint64_t nz = __ballot(key != 0);
      if (lane == 0 && nz) atomicAdd(&s_real, __popcll(nz));
    }
  }
  if (tid == 0) {
    s_prefix = 0;
    s_pmask = 0;
    s_done = 0;
    s_cnt = 0;
  }
  __syncthreads();
  const int kk_sel = (int)min(a.k, (int64_t)s_real);
  if (tid == 0) s_kk = kk_sel;
  __syncthreads();

  if (kk_sel > 0) {
    for (int pass = 0; pass < 8; ++pass) {
      const int shift = 56 - 8 * pass;
      s_hist[tid] = 0;  // TK_THREADS == 256 bins
      __syncthreads();
      const uint64_t prefix = s_prefix, pmask = s_pmask;
      for (int i = tid; i < total; i += TK_THREADS) {
        const uint64_t key = s_keys[i];
        if ((key & pmask) == prefix) atomicAdd(&s_hist[(key >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (wv == 0) {
        // lane l owns bins 255-4l .. 252-4l (descending); find the bin holding
        // the kk-th largest remaining key with a wavefront inclusive scan.
        uint32_t c[4], local = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          c[j] = s_hist[255 - 4 * lane - j];
          local += c[j];
        }
        uint32_t incl = local;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const uint32_t v = __shfl_up(incl, o);
          if (lane >= o) incl += v;
        }
        const uint32_t excl = incl - local;
        const uint32_t kk = (uint32_t)s_kk;
        if (excl < kk && kk <= incl) {
          uint32_t cum = excl;
          int bin = 0;
          uint32_t rem = 0, cnt = 0;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (cnt == 0 && cum + c[j] >= kk) {
              bin = 255 - 4 * lane - j;
              rem = kk - cum;
              cnt = c[j];
            }
            cum += c[j];
          }
          s_prefix = prefix | ((uint64_t)bin << shift);
          s_pmask = pmask | ((uint64_t)0xffu << shift);
          s_kk = (int)rem;
          s_done = (cnt == rem) ? 1 : 0;
        }
      }
      __syncthreads();
      if (s_done) break;
    }

    // winners: (key & pmask) >= prefix; exactly kk_sel of them (keys are
    // unique and the kk_sel-th largest is a real key, above every 0 pad)
    const uint64_t prefix = s_prefix, pmask = s_pmask;
    if constexpr (C::INPLACE) {
      // In place, one 256-key chunk at a time: every key of the chunk is read
      // before any write, and a winner's slot is below the number of keys
      // read so far, so no unread key is overwritten.
      int base = 0;
      for (int i0 = 0; i0 < total; i0 += TK_THREADS) {
        const int i = i0 + tid;
        const uint64_t key = i < total ? s_keys[i] : 0;
        const bool win = i < total && (key & pmask) >= prefix;
        const uint64_t bal = __ballot(win);
        if (lane == 0) s_wcnt[wv] = (int)__popcll(bal);
        __syncthreads();
        int off = base, all = 0;
#pragma unroll
        for (int w = 0; w < TK_THREADS / 64; ++w) {
          off += w < wv ? s_wcnt[w] : 0;
          all += s_wcnt[w];
        }
        if (win) s_keys[off + (int)__popcll(bal & ((1ull << lane) - 1ull))] = key;
        base += all;
        __syncthreads();
      }
    } else {
      for (int i = tid; i < total; i += TK_THREADS) {
        const uint64_t key = s_keys[i];
        if ((key & pmask) >= prefix) {
          const int pos = atomicAdd(&s_cnt, 1);
          if (pos < C::MAX_K) s_sel[pos] = key;
        }
      }
    }
  }
  __syncthreads();
  int P = 1;
  while (P < kk_sel) P <<= 1;
  for (int i = kk_sel + tid; i < P; i += TK_THREADS) s_sel[i] = 0;
  __syncthreads();
  // bitonic sort, descending
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < P / 2; i += TK_THREADS) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const uint64_t x = s_sel[lo], y = s_sel[hi];
        if ((x < y) == desc) {
          s_sel[lo] = y;
          s_sel[hi] = x;
        }
      }
      __syncthreads();
    }
  }
  if (a.keys_out) {
    uint64_t* dst = a.keys_out + ((int64_t)blockIdx.x) * a.k;
    for (int i = tid; i < a.k; i += TK_THREADS) dst[i] = i < kk_sel ? s_sel[i] : 0;
  } else {
    for (int i = tid; i < kk_sel; i += TK_THREADS) {
      const uint64_t key = s_sel[i];
      uint32_t o = (uint32_t)(key >> 32);
      if (!a.largest) o = ~o;
      a.out_s[row * a.old + i] = order_float(o);
      a.out_i[row * a.old + i] = (int64_t)(uint32_t)(~(uint32_t)key);
    }
  }
}

// Tree shape for one call: level-0 groups, lists merged per later group, and
// the workspace (two ping-pong key buffers of rows * groups0 * k keys).
struct TopkPlan {
  int64_t g0, merge, ws_bytes;
};
template <int CLS>
inline TopkPlan topk_plan_cls(int64_t rows, int64_t n, int64_t k) {
  using C = TkCap<CLS>;
  TopkPlan t;
  t.g0 = n <= C::MAX_N ? 1 : (n + C::MAX_N - 1) / C::MAX_N;
  t.merge = k > 0 ? C::MAX_KEYS / k : 1;
  t.ws_bytes = t.g0 > 1 ? 2 * rows * t.g0 * k * (int64_t)sizeof(uint64_t) : 0;
  return t;
}
inline TopkPlan topk_plan(int64_t rows, int64_t n, int64_t k) {
  return topk_class(k) == 0 ? topk_plan_cls<0>(rows, n, k) : topk_plan_cls<1>(rows, n, k);
}
inline int64_t topk_max_n(int64_t k) { return topk_class(k) == 0 ? TkCap<0>::MAX_N : TkCap<1>::MAX_N; }
inline int64_t topk_max_k(int64_t k) { return topk_class(k) == 0 ? TkCap<0>::MAX_K : TkCap<1>::MAX_K; }
// PLAID approximate score, plaid.py:28-79 semantics: one wavefront per doc,
// lane s < Lq keeps the running max of qcs[code, s] over the doc's tokens.
__global__ void __launch_bounds__(256)
    plaid_approx_kernel(const float* __restrict__ qcs, int64_t ncent, int64_t lq, int64_t sc, int64_t sl,
                        const int32_t* __restrict__ codes, int64_t B, int64_t L, int64_t cs,
                        const int64_t* __restrict__ lens, float* __restrict__ out) {
  const int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (b >= B) return;
  int64_t len = lens[b];
  len = len < 0 ? 0 : (len > L ? L : len);
  float total = 0.f;
  for (int64_t s0 = 0; s0 < lq; s0 += 64) {
    const int64_t s = s0 + lane;
    float m = -__builtin_huge_valf();
    if (s < lq) {
      for (int64_t t = 0; t < len; ++t) {
        int64_t code = codes[b * cs + t];
        code = (code >= 0 && code < ncent) ? code : 0;
        m = max_nan(m, qcs[code * sc + s * sl]);
      }
    }
    // a non-finite max (empty doc, NaN or +inf score) contributes 0 (reference.py:119-120)
    float v = (s < lq && __builtin_isfinite(m)) ? m : 0.f;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    total += v;
  }
  if (lane == 0) out[b] = total;
}

// The same score for query-centroid rows of at most 32 fp32 values with unit
// stride and 16-byte aligned rows (the documented qcs = centroids @ Q^T):
// one wavefront per doc; lane (g = lane / 8, q = lane % 8) keeps the running
// maxima of slots 4q .. 4q+3 over the doc's tokens t = 8i + g, so one
// dwordx4 gather instruction reads 8 tokens' whole rows (8 lanes per 128-byte
// row). Per 64 tokens: one coalesced load of their codes (lane l: token l),
// 8 ds_bpermute to hand token 8i + g's code to its group, 8 row gathers.
// At the doc's end the 8 groups' maxima meet (xor 8 by DPP row_ror:8, xor 16
// and 32 by permlane swaps), a non-finite max scores 0, and the slots are
// summed (in lane, then over the 8 lanes of a group).
__global__ void __launch_bounds__(256)
    plaid_approx_rows_kernel(const float* __restrict__ qcs, int64_t ncent, int lq, int64_t sc,
                             const int32_t* __restrict__ codes, int64_t B, int64_t L, int64_t cs,
                             const int64_t* __restrict__ lens, float* __restrict__ out) {
  // wave-uniform doc index and length (so the buffer descriptors are scalar)
  const int64_t b = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63, g = lane >> 3, q = lane & 7;
  if (b >= B) return;
  int64_t len = lens[b];
  len = len < 0 ? 0 : (len > L ? L : len);
  len = __builtin_amdgcn_readfirstlane((int)len);
  constexpr float NEG_INF = -__builtin_huge_valf();
  // raw buffers (untyped, byte range checked): reads past them return 0
  const __amdgpu_buffer_rsrc_t rq =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(qcs), (short)0, (int)(ncent * sc * 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t rc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int32_t*>(codes + b * cs), (short)0, (int)(len * 4), 0x00020000);
  float m[4] = {NEG_INF, NEG_INF, NEG_INF, NEG_INF};
  for (int64_t t0 = 0; t0 < len; t0 += 64) {
    int32_t c = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rc, (uint32_t)((t0 + lane) * 4), 0, 0);
    c = (c >= 0 && c < ncent) ? c : 0;  // out-of-range codes read row 0 (plaid.py:66-67)
    f32x4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int ci = __builtin_amdgcn_ds_bpermute((8 * i + g) * 4, c);
      v[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                           rq, (uint32_t)(ci * sc * 4) + (uint32_t)(q * 16), 0, 0));
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bool ok = t0 + 8 * i + g < len;
#pragma unroll
      for (int k = 0; k < 4; ++k) m[k] = max_nan(m[k], ok ? v[i][k] : NEG_INF);
    }
  }
  auto dpp_ror8 = [](float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false));
  };
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float x = max_nan(m[k], dpp_ror8(m[k]));  // groups g, g ^ 1 (lanes l, l ^ 8)
    auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = max_nan(__uint_as_float(s16[0]), __uint_as_float(s16[1]));  // g ^ 2
    auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = max_nan(__uint_as_float(s32[0]), __uint_as_float(s32[1]));  // g ^ 4
    // empty doc (-inf), NaN or +inf: the slot scores 0 (reference.py:119-120)
    tot += (4 * q + k < lq && __builtin_isfinite(x)) ? x : 0.f;
  }
  // sum over the 8 slot quads (lanes q = 0..7 of group 0, fixed order)
#pragma unroll
  for (int o = 1; o < 8; o <<= 1) tot += __shfl_xor(tot, o);
  if (lane == 0) out[b] = tot;
}

}  // namespace lik

using namespace lik;

extern "C" {

static int topk_validate(const float* scores, int64_t rows, int64_t n, int64_t idx_base, const float* prev_scores,
                         const int64_t* prev_idx, int64_t prev_k, int64_t k, float* out_scores, int64_t* out_idx) {
  if (rows < 0 || n < 0 || prev_k < 0 || k < 0) return LIK_ERR_INVALID;
  if (rows == 0 || k == 0) return LIK_OK;
  // k picks the capacity class; the running list must fit the same class
  if (k > TK_MAX_K || prev_k > topk_max_k(k)) return LIK_ERR_UNSUPPORTED;
  if (k > prev_k + n) return LIK_ERR_INVALID;
  if (n > 0 && !scores) return LIK_ERR_INVALID;
  if (prev_k > 0 && (!prev_scores || !prev_idx)) return LIK_ERR_INVALID;
  if (!out_scores || !out_idx) return LIK_ERR_INVALID;
  if (idx_base < 0 || idx_base + n > 0xffffffffLL) return LIK_ERR_UNSUPPORTED;
  return 1;
}

static int topk_run(const float* scores, int64_t rows, int64_t n, int64_t ld, int64_t idx_base,
                    const float* prev_scores, const int64_t* prev_idx, int64_t prev_k, int64_t prev_ld, int64_t k,
                    int largest, float* out_scores, int64_t* out_idx, int64_t out_ld, void* ws, hipStream_t st) {
  const TopkPlan t = topk_plan(rows, n, k);
  if (rows * t.g0 > 0x7fffffffLL) return LIK_ERR_UNSUPPORTED;
  TopkArgs a{};
  a.scores = scores;
  a.n = n;
  a.ld = ld;
  a.idx_base = idx_base;
  a.prev_s = prev_scores;
  a.prev_i = prev_idx;
  a.pk = prev_k;
  a.pld = prev_ld;
  a.k = k;
  a.largest = largest;
  a.groups = (int)t.g0;
  a.per_group = topk_max_n(k);
  a.out_s = out_scores;
  a.out_i = out_idx;
  a.old = out_ld;
  uint64_t* bufs[2] = {(uint64_t*)ws, ws ? (uint64_t*)ws + rows * t.g0 * k : nullptr};
  a.keys_out = t.g0 > 1 ? bufs[0] : nullptr;
  const bool big = topk_class(k) != 0;
  void (*const level0)(TopkArgs) = big ? topk_select_kernel<1, false> : topk_select_kernel<0, false>;
  void (*const merge)(TopkArgs) = big ? topk_select_kernel<1, true> : topk_select_kernel<0, true>;
  hipLaunchKernelGGL(level0, dim3((unsigned)(rows * t.g0)), dim3(TK_THREADS), 0, st, a);
  int64_t lists = t.g0;
  int cur = 0;
  while (lists > 1) {
    const int64_t groups = (lists + t.merge - 1) / t.merge;
    a.keys_in = bufs[cur];
    a.nin = lists * k;
    a.groups = (int)groups;
    a.per_group = t.merge * k;
    a.keys_out = groups > 1 ? bufs[cur ^ 1] : nullptr;
    hipLaunchKernelGGL(merge, dim3((unsigned)(rows * groups)), dim3(TK_THREADS), 0, st, a);
    lists = groups;
    cur ^= 1;
  }
  return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
}

int lik_topk_merge(const float* scores, int64_t rows, int64_t n, int64_t ld, int64_t idx_base,
                   const float* prev_scores, const int64_t* prev_idx, int64_t prev_k, int64_t prev_ld,
                   int64_t k, int largest, float* out_scores, int64_t* out_idx, int64_t out_ld,
                   lik_stream_t stream) {
  const int v = topk_validate(scores, rows, n, idx_base, prev_scores, prev_idx, prev_k, k, out_scores, out_idx);
  if (v != 1) return v;
  if (n > topk_max_n(k)) return LIK_ERR_UNSUPPORTED;
  return topk_run(scores, rows, n, ld, idx_base, prev_scores, prev_idx, prev_k, prev_ld, k, largest, out_scores,
                  out_idx, out_ld, nullptr, (hipStream_t)stream);
}

size_t lik_topk_select_workspace_size(int64_t rows, int64_t n, int64_t k) {
  if (rows < 0 || n < 0 || k < 0) return 0;
  return (size_t)topk_plan(rows, n, k).ws_bytes;
}

int lik_topk_select(const float* scores, int64_t rows, int64_t n, int64_t ld, int64_t idx_base,
                    const float* prev_scores, const int64_t* prev_idx, int64_t prev_k, int64_t prev_ld, int64_t k,
                    int largest, float* out_scores, int64_t* out_idx, int64_t out_ld, void* workspace,
                    size_t workspace_bytes, lik_stream_t stream) {
  const int v = topk_validate(scores, rows, n, idx_base, prev_scores, prev_idx, prev_k, k, out_scores, out_idx);
  if (v != 1) return v;
  const TopkPlan t = topk_plan(rows, n, k);
  if (t.ws_bytes > 0 && (!workspace || workspace_bytes < (size_t)t.ws_bytes)) return LIK_ERR_WORKSPACE;
  return topk_run(scores, rows, n, ld, idx_base, prev_scores, prev_idx, prev_k, prev_ld, k, largest, out_scores,
                  out_idx, out_ld, workspace, (hipStream_t)stream);
}

int lik_plaid_approx_score(const float* qcs, int64_t n_centroids, int64_t lq, int64_t qcs_stride_c,
                           int64_t qcs_stride_l, const int32_t* codes, int64_t B, int64_t max_len,
                           int64_t codes_stride_b, const int64_t* doc_lengths, float* out,
                           lik_stream_t stream) {
  if (B < 0 || lq < 0 || n_centroids < 1 || max_len < 0) return LIK_ERR_INVALID;
  if (B == 0) return LIK_OK;
  if (!qcs || !codes || !doc_lengths || !out) return LIK_ERR_INVALID;
  if ((B + 3) / 4 > 0x7fffffffLL) return LIK_ERR_UNSUPPORTED;
  // rows of <= 32 unit-stride, 16-byte aligned scores: whole rows per gather
  const bool rows = lq > 0 && lq <= 32 && qcs_stride_l == 1 && qcs_stride_c % 4 == 0 &&
                    ((uintptr_t)qcs) % 16 == 0 && n_centroids * qcs_stride_c * 4 < (int64_t)0xffffffffLL &&
                    max_len * 4 < (int64_t)0xffffffffLL;
  if (rows)
    hipLaunchKernelGGL(plaid_approx_rows_kernel, dim3((unsigned)((B + 3) / 4)), dim3(256), 0, (hipStream_t)stream,
                       qcs, n_centroids, (int)lq, qcs_stride_c, codes, B, max_len, codes_stride_b, doc_lengths, out);
  else
    hipLaunchKernelGGL(plaid_approx_kernel, dim3((unsigned)((B + 3) / 4)), dim3(256), 0, (hipStream_t)stream, qcs,
                       n_centroids, lq, qcs_stride_c, qcs_stride_l, codes, B, max_len, codes_stride_b, doc_lengths,
                       out);
  return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
}

}  // extern "C"
