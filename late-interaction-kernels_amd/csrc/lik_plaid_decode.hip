// PLAID token decode for gfx950: centroid code + n-bit residual fields ->
// (optionally L2-normalised) bf16 / fp16 token rows in HBM.
//
// emb[f] = centroids[code, f] + bucket_weights[field_f], field_f the nbits-bit
// field f of the token's packed residual row, little-endian within each
// byte (reference.py:124-139, plaid.py:240-274). Out-of-range codes decode
// as centroid 0 and out-of-range bucket codes as the last bucket, as in the
// fused tile kernel.
//
// The arithmetic is the fused kernel's staging pass, element for element:
// the same fp32 adds, the same per-lane fma chain over 8 elements, the same
// xor-shuffle reduction over the lanes of a row (lane group = padded dim / 8,
// zeros past the dim), the same rounding. A decoded row is therefore
// bitwise the row the fused kernel would have put in LDS, so decode-then-
// dense-MaxSim and fused decode+MaxSim give identical scores.
//
// Work: one lane per 8 embedding elements (16 bytes out); a 256-thread
// workgroup covers 4 x 256 / (dpad / 8) tokens (four passes, loads first). Per token it reads 4 bytes of
// code, dim*nbits/8 bytes of residual and one centroid row (L2 / MALL
// resident for typical tables), and writes dim*2 bytes: an HBM-bound kernel.
#include "lik_common.h"

namespace lik {

// Tokens per lane group: a workgroup makes kDecodeTPT passes of 256 / LPT
// tokens, and issues the loads of all of them (codes, then centroid rows and
// residual bits) before it decodes the first: with one token per lane group
// each wave held 1 KB of rows in flight behind two dependent load latencies
// (code, then row), too little to cover them.
constexpr int kDecodeTPT = 4;

template <int LPT, int CD, int OUTK>
__global__ void __launch_bounds__(256)
    plaid_decode_kernel(const int32_t* __restrict__ codes, const uint8_t* __restrict__ res, int64_t res_st,
                        const char* __restrict__ cent, int64_t cent_sb, int64_t ncent,
                        const float* __restrict__ bw, int nb, int nbits, int dim, int normalize,
                        uint16_t* __restrict__ out, int64_t out_stride, int64_t ntok, float* __restrict__ inv_out,
                        int rec) {
  constexpr int TPB = 256 / LPT;  // tokens per pass
  constexpr int TPT = kDecodeTPT;
  constexpr int CSZ = CD == EK_F32 ? 4 : 2;
  constexpr int NCV = CD == EK_F32 ? 2 : 1;
  __shared__ float s_bw[256];
  for (int i = threadIdx.x; i < 256; i += 256) s_bw[i] = i < nb ? bw[i] : 0.f;
  __syncthreads();
  const int cc = threadIdx.x % LPT;  // 8-element chunk of the row
  const int64_t tok0 = (int64_t)blockIdx.x * (TPB * TPT) + threadIdx.x / LPT;
  int64_t code[TPT];
#pragma unroll
  for (int k = 0; k < TPT; ++k) {
    const int64_t tok = tok0 + (int64_t)k * TPB;
    int64_t c = tok < ntok ? codes[tok] : 0;
    code[k] = (c < 0 || c >= ncent) ? 0 : c;
  }
  u32x4 cv4[TPT][NCV];
  uint64_t bits[TPT];
#pragma unroll
  for (int k = 0; k < TPT; ++k) {
    const int64_t tok = tok0 + (int64_t)k * TPB;
    const bool live = tok < ntok && cc * 8 < dim;
    bits[k] = 0;
#pragma unroll
    for (int v = 0; v < NCV; ++v) cv4[k][v] = u32x4{0u, 0u, 0u, 0u};
    if (live) {
      const char* crow = cent + code[k] * cent_sb + (int64_t)cc * 8 * CSZ;
      const uint8_t* rrow = res + tok * res_st + (int64_t)cc * nbits;
      if (nbits == 2) bits[k] = *(const uint16_t*)rrow;
      else if (nbits == 4) bits[k] = *(const uint32_t*)rrow;
      else bits[k] = *(const uint64_t*)rrow;
      cv4[k][0] = *(const u32x4*)crow;
      if constexpr (CD == EK_F32) cv4[k][1] = *(const u32x4*)(crow + 16);
    }
  }
#pragma unroll
  for (int k = 0; k < TPT; ++k) {
    const int64_t tok = tok0 + (int64_t)k * TPB;
    const bool tok_ok = tok < ntok;
    const bool live = tok_ok && cc * 8 < dim;
    float x8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) x8[e] = 0.f;
    if (live) {
      const uint32_t bmask = (1u << nbits) - 1u;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float cv;
        if constexpr (CD == EK_F32) cv = __uint_as_float(cv4[k][e >> 2][e & 3]);
        else if constexpr (CD == EK_BF16)
          cv = (e & 1) ? bf16hi_to_f32(cv4[k][0][e >> 1]) : bf16lo_to_f32(cv4[k][0][e >> 1]);
        else
          cv = f16_to_f32((uint16_t)((e & 1) ? (cv4[k][0][e >> 1] >> 16) : (cv4[k][0][e >> 1] & 0xffffu)));
        uint32_t bc = (uint32_t)(bits[k] >> (e * nbits)) & bmask;
        bc = bc < (uint32_t)nb ? bc : (uint32_t)(nb - 1);
        x8[e] = (cc * 8 + e) < dim ? cv + s_bw[bc] : 0.f;
      }
    }
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf(x8[e], x8[e], ss);
#pragma unroll
    for (int o = 1; o < LPT; o <<= 1) ss += __shfl_xor(ss, o);
    // norms-only mode (out == null): the token's inverse norm, 1 / max(||x||, 1e-12),
    // alone or after the token's code as an 8-byte (code, norm) record
    if (inv_out) {
      if (tok_ok && cc == 0) {
        if (rec)
          *(uint2*)(inv_out + 2 * tok) = uint2{(uint32_t)codes[tok], __float_as_uint(inv_norm(ss))};
        else
          inv_out[tok] = inv_norm(ss);
      }
      continue;
    }
    const float sc = normalize ? inv_norm(ss) : 1.f;
    if (live) {
      u32x4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (OUTK == EK_F16)
          w[e] = f32_to_f16_bits(x8[2 * e] * sc) | (f32_to_f16_bits(x8[2 * e + 1] * sc) << 16);
        else
          w[e] = f32_to_bf16_bits(x8[2 * e] * sc) | (f32_to_bf16_bits(x8[2 * e + 1] * sc) << 16);
      }
      *(u32x4*)(out + tok * out_stride + cc * 8) = w;
    }
  }
}

template <int LPT, int CD>
int launch_decode_cd(int outk, const lik_plaid_docs_t* d, const int32_t* codes, const uint8_t* res, int norm,
                     uint16_t* out, int64_t out_stride, int64_t ntok, float* inv_out, int rec, hipStream_t s) {
  constexpr int TPW = 256 / LPT * kDecodeTPT;  // tokens per workgroup
  const int ceb = CD == EK_F32 ? 4 : 2;
  const dim3 grid((unsigned)((ntok + TPW - 1) / TPW));
  if (outk == EK_F16)
    hipLaunchKernelGGL((plaid_decode_kernel<LPT, CD, EK_F16>), grid, dim3(256), 0, s, codes, res, d->res_stride_tok,
                       (const char*)d->centroids, d->cent_stride * ceb, d->n_centroids, d->bucket_weights,
                       d->n_buckets, d->nbits, d->dim, norm, out, out_stride, ntok, inv_out, rec);
  else
    hipLaunchKernelGGL((plaid_decode_kernel<LPT, CD, EK_BF16>), grid, dim3(256), 0, s, codes, res, d->res_stride_tok,
                       (const char*)d->centroids, d->cent_stride * ceb, d->n_centroids, d->bucket_weights,
                       d->n_buckets, d->nbits, d->dim, norm, out, out_stride, ntok, inv_out, rec);
  return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
}

template <int LPT>
int launch_decode(int outk, const lik_plaid_docs_t* d, const int32_t* codes, const uint8_t* res, int norm,
                  uint16_t* out, int64_t out_stride, int64_t ntok, float* inv_out, hipStream_t s, int rec = 0) {
  switch (d->centroid_dtype) {
    case LIK_BF16: return launch_decode_cd<LPT, EK_BF16>(outk, d, codes, res, norm, out, out_stride, ntok, inv_out, rec, s);
    case LIK_F16: return launch_decode_cd<LPT, EK_F16>(outk, d, codes, res, norm, out, out_stride, ntok, inv_out, rec, s);
    case LIK_F32: return launch_decode_cd<LPT, EK_F32>(outk, d, codes, res, norm, out, out_stride, ntok, inv_out, rec, s);
    default: return LIK_ERR_UNSUPPORTED;
  }
}

// out[i] = in[i] with its 8 bits reversed, 4 bytes per thread: reversing a
// 32-bit word and swapping its bytes back reverses the bits inside each byte.
__global__ void __launch_bounds__(256) reverse_bits_kernel(const uint8_t* in, uint8_t* out, int64_t n) {
  const int64_t w = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t b = w * 4;
  if (b + 4 <= n) {
    const uint32_t v = *(const uint32_t*)(in + b);
    *(uint32_t*)(out + b) = __builtin_bswap32(__builtin_bitreverse32(v));
  } else {
    for (int64_t i = b; i < n; ++i) out[i] = __builtin_bitreverse8(in[i]);
  }
}

}  // namespace lik

using namespace lik;

extern "C" int lik_residual_reverse_bits(const uint8_t* in, uint8_t* out, int64_t nbytes, lik_stream_t stream) {
  if (nbytes < 0 || (nbytes > 0 && (!in || !out))) return LIK_ERR_INVALID;
  if (((uintptr_t)in) % 4 || ((uintptr_t)out) % 4) return LIK_ERR_UNSUPPORTED;
  if (nbytes == 0) return LIK_OK;
  const int64_t words = (nbytes + 3) / 4;
  if ((words + 255) / 256 > 0x7fffffffLL) return LIK_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(reverse_bits_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, (hipStream_t)stream, in,
                     out, nbytes);
  return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
}

extern "C" int lik_plaid_decode(const lik_plaid_docs_t* docs, int64_t tok_begin, int64_t tok_end, uint32_t flags,
                                int32_t out_dtype, void* out, int64_t out_stride, lik_stream_t stream) {
  if (!docs || tok_begin < 0 || tok_end < tok_begin) return LIK_ERR_INVALID;
  if (docs->nbits != 2 && docs->nbits != 4 && docs->nbits != 8) return LIK_ERR_INVALID;
  if (docs->dim <= 0 || docs->dim % 8 != 0) return LIK_ERR_INVALID;
  if (docs->n_buckets < 1 || docs->n_buckets > 256 || !docs->bucket_weights) return LIK_ERR_INVALID;
  if (out_dtype != LIK_BF16 && out_dtype != LIK_F16) return LIK_ERR_UNSUPPORTED;
  if (docs->res_stride_tok * 8 < (int64_t)docs->dim * docs->nbits) return LIK_ERR_INVALID;
  if (out_stride < docs->dim || (out_stride * 2) % 16 != 0 || ((uintptr_t)out) % 16 != 0) return LIK_ERR_UNSUPPORTED;
  const int64_t ntok = tok_end - tok_begin;
  if (ntok == 0) return LIK_OK;
  if (!out || !docs->codes || !docs->residuals || !docs->centroids || docs->n_centroids < 1) return LIK_ERR_INVALID;
  const int ceb = docs->centroid_dtype == LIK_F32 ? 4 : 2;
  if (((uintptr_t)docs->centroids) % 16 != 0 || (docs->cent_stride * ceb) % 16 != 0) return LIK_ERR_UNSUPPORTED;
  if (((uintptr_t)docs->residuals) % 8 != 0 || docs->res_stride_tok % docs->nbits != 0) return LIK_ERR_UNSUPPORTED;
  if (ntok > (int64_t)0x7fffffff * 8) return LIK_ERR_UNSUPPORTED;
  const int32_t* codes = docs->codes + tok_begin;
  const uint8_t* res = docs->residuals + tok_begin * docs->res_stride_tok;
  const int norm = (flags & LIK_NORMALIZE) ? 1 : 0;
  const int outk = out_dtype == LIK_F16 ? EK_F16 : EK_BF16;
  uint16_t* o = (uint16_t*)out;
  hipStream_t s = (hipStream_t)stream;
  // lane group per token = padded dim / 8 (the fused kernel's row reduction width)
  if (docs->dim <= 64) return launch_decode<8>(outk, docs, codes, res, norm, o, out_stride, ntok, nullptr, s);
  if (docs->dim <= 128) return launch_decode<16>(outk, docs, codes, res, norm, o, out_stride, ntok, nullptr, s);
  if (docs->dim <= 256) return launch_decode<32>(outk, docs, codes, res, norm, o, out_stride, ntok, nullptr, s);
  return LIK_ERR_UNSUPPORTED;
}

namespace {
// inverse norms (rec = 0: 4 bytes per token) or (code, inverse norm) records
// (rec = 1: 8 bytes per token) of tokens [tok_begin, tok_end), indexed by
// absolute token
int token_norms(const lik_plaid_docs_t* docs, int64_t tok_begin, int64_t tok_end, float* inv, int rec,
                lik_stream_t stream) {
  if (!docs || tok_begin < 0 || tok_end < tok_begin) return LIK_ERR_INVALID;
  if (docs->nbits != 2 && docs->nbits != 4 && docs->nbits != 8) return LIK_ERR_INVALID;
  if (docs->dim <= 0 || docs->dim % 8 != 0) return LIK_ERR_INVALID;
  if (docs->n_buckets < 1 || docs->n_buckets > 256 || !docs->bucket_weights) return LIK_ERR_INVALID;
  if (docs->res_stride_tok * 8 < (int64_t)docs->dim * docs->nbits) return LIK_ERR_INVALID;
  const int64_t ntok = tok_end - tok_begin;
  if (ntok == 0) return LIK_OK;
  if (!inv || !docs->codes || !docs->residuals || !docs->centroids || docs->n_centroids < 1) return LIK_ERR_INVALID;
  const int ceb = docs->centroid_dtype == LIK_F32 ? 4 : 2;
  if (((uintptr_t)docs->centroids) % 16 != 0 || (docs->cent_stride * ceb) % 16 != 0) return LIK_ERR_UNSUPPORTED;
  if (((uintptr_t)docs->residuals) % 8 != 0 || docs->res_stride_tok % docs->nbits != 0) return LIK_ERR_UNSUPPORTED;
  if (ntok > (int64_t)0x7fffffff * 8) return LIK_ERR_UNSUPPORTED;
  const int32_t* codes = docs->codes + tok_begin;
  const uint8_t* res = docs->residuals + tok_begin * docs->res_stride_tok;
  if (rec && ((uintptr_t)inv) % 8) return LIK_ERR_UNSUPPORTED;
  // (the kernel indexes its output from the range's first token)
  float* o = inv + (rec ? 2 : 1) * tok_begin;
  hipStream_t s = (hipStream_t)stream;
  if (docs->dim <= 64) return launch_decode<8>(EK_BF16, docs, codes, res, 1, nullptr, 0, ntok, o, s, rec);
  if (docs->dim <= 128) return launch_decode<16>(EK_BF16, docs, codes, res, 1, nullptr, 0, ntok, o, s, rec);
  if (docs->dim <= 256) return launch_decode<32>(EK_BF16, docs, codes, res, 1, nullptr, 0, ntok, o, s, rec);
  return LIK_ERR_UNSUPPORTED;
}
}  // namespace

extern "C" int lik_plaid_token_norms(const lik_plaid_docs_t* docs, int64_t tok_begin, int64_t tok_end, float* inv,
                                     lik_stream_t stream) {
  return token_norms(docs, tok_begin, tok_end, inv, 0, stream);
}

extern "C" int lik_plaid_token_records(const lik_plaid_docs_t* docs, int64_t tok_begin, int64_t tok_end,
                                       lik_plaid_token_t* rec, lik_stream_t stream) {
  return token_norms(docs, tok_begin, tok_end, (float*)rec, 1, stream);
}
