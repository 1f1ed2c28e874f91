// Chunked top-k merge and PLAID approximate scoring for gfx950.
//
// Top-k: each (score, index) candidate becomes one 64-bit key
//   key = order(score) << 32 | ~index
// where order() is the monotone float->uint32 map (descending scores map to
// descending keys; for largest=False the score part is complemented). Keys
// are unique, and "larger key" == "better score, then lower index", so the k
// best candidates are exactly the k largest keys. One workgroup per row finds
// the k-th largest key by an 8-pass MSB-first radix select over LDS-resident
// keys (256-bin histograms), compacts the winners and bitonic-sorts them.
// This replaces topk.py:41-86 / retrieve.py:278-305 (torch.topk + cat +
// gather per chunk) and pins the tie order torch.topk leaves unspecified.
#include "lik_common.h"

namespace lik {

constexpr int TK_THREADS = 256;
constexpr int TK_MAX_N = 4096;  // new candidates per call
constexpr int TK_MAX_K = 1024;
constexpr int TK_MAX_KEYS = TK_MAX_N + TK_MAX_K;

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

__global__ void __launch_bounds__(TK_THREADS)
    topk_merge_kernel(const float* __restrict__ scores, int64_t n, int64_t ld, int64_t idx_base,
                      const float* prev_s, const int64_t* prev_i, int64_t pk, int64_t pld, int64_t k,
                      int largest, float* out_s, int64_t* out_i, int64_t old) {
  __shared__ uint64_t s_keys[TK_MAX_KEYS];
  __shared__ uint64_t s_sel[TK_MAX_K];
  __shared__ uint32_t s_hist[256];
  __shared__ uint64_t s_prefix, s_pmask;
  __shared__ int s_kk, s_done, s_cnt;

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t row = blockIdx.x;
  const int total = (int)(pk + n);

  for (int i = tid; i < total; i += TK_THREADS) {
    uint64_t key;
    if (i < pk) {
      key = make_key(prev_s[row * pld + i], (uint32_t)prev_i[row * pld + i], largest);
    } else {
      const int64_t c = i - pk;
      key = make_key(scores[row * ld + c], (uint32_t)(idx_base + c), largest);
    }
    s_keys[i] = key;
  }
  if (tid == 0) {
    s_prefix = 0;
    s_pmask = 0;
    s_kk = (int)k;
    s_done = 0;
    s_cnt = 0;
  }
  __syncthreads();

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

  // winners: (key & pmask) >= prefix; exactly k of them
  const uint64_t prefix = s_prefix, pmask = s_pmask;
  for (int i = tid; i < total; i += TK_THREADS) {
    const uint64_t key = s_keys[i];
    if ((key & pmask) >= prefix) {
      const int pos = atomicAdd(&s_cnt, 1);
      if (pos < TK_MAX_K) s_sel[pos] = key;
    }
  }
  __syncthreads();
  int P = 1;
  while (P < k) P <<= 1;
  for (int i = (int)k + tid; i < P; i += TK_THREADS) s_sel[i] = 0;
  __syncthreads();
  // bitonic sort, descending
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < P / 2; i += TK_THREADS) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const uint64_t a = s_sel[lo], b = s_sel[hi];
        if ((a < b) == desc) {
          s_sel[lo] = b;
          s_sel[hi] = a;
        }
      }
      __syncthreads();
    }
  }
  for (int i = tid; i < k; i += TK_THREADS) {
    const uint64_t key = s_sel[i];
    uint32_t o = (uint32_t)(key >> 32);
    if (!largest) o = ~o;
    out_s[row * old + i] = order_float(o);
    out_i[row * old + i] = (int64_t)(uint32_t)(~(uint32_t)key);
  }
}

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
        m = fmaxf(m, qcs[code * sc + s * sl]);
      }
    }
    float v = (s < lq && m != -__builtin_huge_valf()) ? m : 0.f;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    total += v;
  }
  if (lane == 0) out[b] = total;
}

}  // namespace lik

using namespace lik;

extern "C" {

int lik_topk_merge(const float* scores, int64_t rows, int64_t n, int64_t ld, int64_t idx_base,
                   const float* prev_scores, const int64_t* prev_idx, int64_t prev_k, int64_t prev_ld,
                   int64_t k, int largest, float* out_scores, int64_t* out_idx, int64_t out_ld,
                   lik_stream_t stream) {
  if (rows < 0 || n < 0 || prev_k < 0 || k < 0) return LIK_ERR_INVALID;
  if (rows == 0 || k == 0) return LIK_OK;
  if (n > TK_MAX_N || k > TK_MAX_K || prev_k > TK_MAX_K) return LIK_ERR_UNSUPPORTED;
  if (k > prev_k + n) return LIK_ERR_INVALID;
  if (n > 0 && !scores) return LIK_ERR_INVALID;
  if (prev_k > 0 && (!prev_scores || !prev_idx)) return LIK_ERR_INVALID;
  if (!out_scores || !out_idx) return LIK_ERR_INVALID;
  if (idx_base < 0 || idx_base + n > 0xffffffffLL) return LIK_ERR_UNSUPPORTED;
  if (rows > 0x7fffffffLL) return LIK_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(topk_merge_kernel, dim3((unsigned)rows), dim3(TK_THREADS), 0, (hipStream_t)stream, scores,
                     n, ld, idx_base, prev_scores, prev_idx, prev_k, prev_ld, k, largest, out_scores, out_idx,
                     out_ld);
  return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
}

int lik_plaid_approx_score(const float* qcs, int64_t n_centroids, int64_t lq, int64_t qcs_stride_c,
                           int64_t qcs_stride_l, const int32_t* codes, int64_t B, int64_t max_len,
                           int64_t codes_stride_b, const int64_t* doc_lengths, float* out,
                           lik_stream_t stream) {
  if (B < 0 || lq < 0 || n_centroids < 1 || max_len < 0) return LIK_ERR_INVALID;
  if (B == 0) return LIK_OK;
  if (!qcs || !codes || !doc_lengths || !out) return LIK_ERR_INVALID;
  hipLaunchKernelGGL(plaid_approx_kernel, dim3((unsigned)((B + 3) / 4)), dim3(256), 0, (hipStream_t)stream, qcs,
                     n_centroids, lq, qcs_stride_c, qcs_stride_l, codes, B, max_len, codes_stride_b, doc_lengths,
                     out);
  return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
}

}  // extern "C"
