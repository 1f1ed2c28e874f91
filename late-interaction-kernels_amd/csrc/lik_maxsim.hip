// MaxSim forward for gfx950: dense / KD / packed (varlen) / pair-list / fp8 /
// PLAID-residual documents, one kernel family.
//
// Work decomposition. A workgroup of W wavefronts owns a block of COLS =
// W*NSUB*32 query tokens ("columns"), held for the workgroup's lifetime in
// VGPRs as MFMA B-fragments, and walks a contiguous range of documents in
// 32-token tiles. Each tile is staged once through LDS (with the optional
// per-token L2 norm, mask bias and, for PLAID, the centroid+residual decode
// fused into the staging pass) and then multiplied by every wavefront
// against its own NSUB column blocks (v_mfma_f32_32x32x16_bf16/f16, or
// v_mfma_scale_f32_32x32x64_f8f6f4 for fp8). Doc tokens are the MFMA rows,
// so the max over doc tokens is an in-lane max over the 16 accumulator
// registers plus one lane^32 exchange at the end of a document; the
// [Nq, Nd, Lq, Ld] similarity tensor never exists, not even per tile in LDS.
// At a document's end the per-column maxima go through LDS and are summed
// per query in a fixed order (bitwise deterministic, no atomics).
//
// Semantics follow late_interaction_kernels/reference.py:26-98 (dense),
// 142-179 (residual), 213-245 (varlen), 248-269 (pairs): a doc-side mask
// removes tokens from the max, a query-side mask from the sum, a max over no
// valid token (or a non-finite max) contributes 0, normalise is
// x / max(||x||, 1e-12).
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include <mutex>


#include "lik_params.h"

namespace lik {


// Per-document summary of a boolean mask: extent = last kept token + 1,
// holes = some token inside [0, extent) is dropped, and one 32-bit
// row-validity word per 32-token tile (bit r = token 32*t + r kept), which
// the tile kernel applies in its epilogue. One wavefront per doc; each pass
// covers two tiles (lanes 0-31 and 32-63) with one ballot.
__global__ void __launch_bounds__(256) doc_extent_kernel(const int8_t* mask, int64_t msn, int64_t msl,
                                                         int64_t n, int64_t L, const int32_t* lengths,
                                                         int32_t* extent, uint8_t* holes, uint32_t* tbits,
                                                         int64_t tbits_sn) {
  const int64_t j = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (j >= n) return;
  int64_t Lj = L;
  if (lengths) {
    const int64_t l = lengths[j];
    Lj = l < 0 ? 0 : (l > L ? L : l);
  }
  int last = -1, cnt = 0;
  for (int64_t t0 = 0; t0 < tbits_sn * 32; t0 += 64) {
    const int64_t t = t0 + lane;
    const bool keep = t < Lj && mask[j * msn + t * msl] != 0;
    if (keep) {
      last = (int)t;
      ++cnt;
    }
    const uint64_t bal = __ballot(keep);
    const int64_t tile = t0 >> 5;
    if (lane == 0 && tile < tbits_sn) tbits[j * tbits_sn + tile] = (uint32_t)bal;
    if (lane == 32 && tile + 1 < tbits_sn) tbits[j * tbits_sn + tile + 1] = (uint32_t)(bal >> 32);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    last = max(last, __shfl_xor(last, o));
    cnt += __shfl_xor(cnt, o);
  }
  if (lane == 0) {
    extent[j] = last + 1;
    holes[j] = (uint8_t)(cnt != last + 1);
  }
}

// The same summary for masks whose token bytes are contiguous (stride 1),
// with 4-byte-aligned rows, L <= 1024 and the whole mask under 4 GB. The
// byte-per-lane form spends ~90 instructions of a 64-lane wavefront per doc
// (and one load round trip per doc); here 16 lanes take a doc, 4 docs per
// wavefront, and lane q reads tokens 16 q .. 16 q + 15 of each 256-token pass
// as four dwords, all of a wavefront's loads issued before any is used. The
// nonzero bytes of a dword become 4 bits by an or-fold and one multiply. The
// loads go through a buffer resource that ends at the mask's last byte (a
// dword past it reads as 0; bytes past a doc's length are dropped by the
// length test).
__device__ __forceinline__ uint32_t nonzero_bytes4(uint32_t x) {
  uint32_t y = x | (x >> 4);
  y |= y >> 2;
  y |= y >> 1;
  y &= 0x01010101u;  // bit 8 k: byte k is nonzero
  // bit 8 k -> bit 24 + k (the other products land below bit 24 without carries)
  return ((y * 0x01020408u) >> 24) & 0xfu;
}

__global__ void __launch_bounds__(256) doc_extent_w4_kernel(const int8_t* mask, int64_t msn, uint32_t mbytes,
                                                            int64_t n, int L, const int32_t* lengths,
                                                            int32_t* extent, uint8_t* holes, uint32_t* tbits,
                                                            int tbits_sn) {
  constexpr int NP = 4;  // 256-token passes (L <= 1024)
  const int lane = threadIdx.x & 63, q = lane & 15;
  const int64_t j = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 4 + (lane >> 4);
  const int np = (L + 255) >> 8;  // passes that hold tokens (uniform)
  int Lj = j < n ? L : 0;
  if (lengths && j < n) {
    const int l = lengths[j];
    Lj = l < 0 ? 0 : (l > L ? L : l);
  }
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(mask), (short)0, (int)mbytes, 0x00020000);
  const uint32_t row = j < n ? (uint32_t)(j * msn) : 0u;
  uint32_t w[NP][4];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = p * 256 + q * 16 + 4 * i;
      w[p][i] = (p < np && t < Lj) ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs, row + (uint32_t)t, 0, 0) : 0u;
    }
  }
  int last = -1, cnt = 0;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    if (p >= np) break;
    const int t = p * 256 + q * 16;
    uint32_t m = nonzero_bytes4(w[p][0]) | (nonzero_bytes4(w[p][1]) << 4) | (nonzero_bytes4(w[p][2]) << 8) |
                 (nonzero_bytes4(w[p][3]) << 12);
    const int room = Lj - t;  // tokens of this lane's sixteen that lie inside the doc
    m &= room >= 16 ? 0xffffu : (room <= 0 ? 0u : (1u << room) - 1u);
    if (m) last = t + 31 - __builtin_clz(m);
    cnt += __builtin_popcount(m);
    // tile p * 8 + q / 2 (32 tokens) = the 16-bit groups of lanes q, q ^ 1
    uint32_t v = m << (16 * (q & 1));
    v |= __shfl_xor(v, 1);
    const int tile = p * 8 + (q >> 1);
    if (j < n && (q & 1) == 0 && tile < tbits_sn) tbits[j * tbits_sn + tile] = v;
  }
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) {
    last = max(last, __shfl_xor(last, o));
    cnt += __shfl_xor(cnt, o);
  }
  if (j < n && q == 0) {
    extent[j] = last + 1;
    holes[j] = (uint8_t)(cnt != last + 1);
  }
}

// a[i] = v for i < n (used to mark argmax entries "no winner" before a training forward).
__global__ void __launch_bounds__(256) fill_i32_kernel(int32_t* a, int64_t n, int32_t v) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) a[i] = v;
}

// Doc-token normalisation ahead of the tile kernel: out[j, t] = D[j, t] /
// max(||D[j, t]||, 1e-12), rounded once to the input type, into a contiguous
// [n, L, dim] buffer. LPR lanes per row (the row's 16-byte chunks, zeros past
// dim), each summing its chunk's squares in element order, then an xor-
// shuffle over the row's lanes: the arithmetic of the tile kernel's commit,
// so the rows are bitwise those it would have normalised in LDS.
template <int EK, int LPR>
__global__ void __launch_bounds__(256) norm_rows_kernel(const char* x, int64_t sn, int64_t sl, int64_t n, int64_t L,
                                                        int dim, char* out) {
  constexpr int EPC = 8;  // bf16 / fp16 elements per chunk
  const int64_t r = ((int64_t)blockIdx.x * 256 + threadIdx.x) / LPR;
  const int cc = threadIdx.x % LPR;
  const bool ok = r < n * L;
  const bool live = ok && cc * EPC < dim;
  u32x4 v = {0u, 0u, 0u, 0u};
  if (live) v = *(const u32x4*)(x + (r / L) * sn + (r % L) * sl + (int64_t)cc * 16);
  float ss = chunk_sumsq<EK>(v);
#pragma unroll
  for (int o = 1; o < LPR; o <<= 1) ss += __shfl_xor(ss, o);
  const float sc = inv_norm(ss);
  if (!live) return;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if constexpr (EK == EK_BF16)
      v[e] = f32_to_bf16_bits(bf16lo_to_f32(v[e]) * sc) | (f32_to_bf16_bits(bf16hi_to_f32(v[e]) * sc) << 16);
    else
      v[e] = f32_to_f16_bits(f16_to_f32((uint16_t)(v[e] & 0xffffu)) * sc) |
             (f32_to_f16_bits(f16_to_f32((uint16_t)(v[e] >> 16)) * sc) << 16);
  }
  *(u32x4*)(out + r * (int64_t)dim * 2 + (int64_t)cc * 16) = v;
}

// out[q, j] = sum_c part[q*nc + c, j], c ascending.
__global__ void __launch_bounds__(256) unit_sum_kernel(const float* part, int64_t nq, int nc, int64_t nd,
                                                       float* out, int64_t osq, int64_t osd) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nq * nd) return;
  const int64_t q = i / nd, j = i - q * nd;
  float s = 0.f;
  for (int c = 0; c < nc; ++c) s += part[(q * nc + c) * nd + j];
  out[q * osq + j * osd] = s;
}

}  // namespace lik

// ============================================================================
// Host side: validation, configuration and launch.
// ============================================================================
using namespace lik;

namespace {

struct Cfg {
  int W, NSUB;
};
// Column-block configurations, smallest first. The largest ones put two
// wavefronts on each SIMD (8 per workgroup) so one wave's bookkeeping hides
// under the other's MFMAs: 8x2 for 16-bit types; fp8 (half the fragment
// registers, twice the MFMA rate) goes to 8x4 to amortise the per-tile work
// over more MFMAs.
// At equal column count the wider workgroup comes first: more waves share
// each tile's staging work.
constexpr Cfg kCfgs[] = {{1, 1}, {1, 2}, {4, 1}, {1, 4}, {8, 1}, {4, 2}, {8, 2}, {4, 4}, {8, 4}};
constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

int elem_bytes(int dt) { return dt == LIK_F32 ? 4 : (dt == LIK_FP8_E4M3 ? 1 : 2); }

int pick_dpad(int dt, int dim) {
  const int opts[] = {64, 128, 256, 512};
  for (int o : opts)
    if (dim <= o) {
      if (dt == LIK_F32 && o > 256) return -1;
      if (dt == LIK_FP8_E4M3 && o > 256) return -1;
      return o;
    }
  return -1;
}

// VGPRs of query (B) fragments one 32-column block holds per lane.
int bfrag_regs(int dt, int dpad) {
  const int fe = dt == LIK_FP8_E4M3 ? 32 : 8;
  const int cb = dt == LIK_FP8_E4M3 ? 1 : 2;
  const int ks = dpad / (2 * fe);
  const int fv = fe * cb / 16;
  return ks * fv * 4 * (dt == LIK_F32 ? 2 : 1);
}

int max_nsub(int dt, int dpad) {
  int n = 128 / bfrag_regs(dt, dpad);
  return n > 4 ? 4 : n;
}

// A token scale with both strides 0 is one per-tensor scale: it is folded
// into the score scale at the epilogue (read from device memory there)
// instead of scaling rows.
bool tensor_scale(const lik_seqs_t& s) { return s.token_scale && s.scale_stride_n == 0 && s.scale_stride_l == 0; }
bool row_scale(const lik_seqs_t* s) { return s->token_scale && !tensor_scale(*s); }

SeqDev to_dev(const lik_seqs_t& s) {
  SeqDev d;
  const int eb = elem_bytes(s.dtype);
  d.data = (const char*)s.data;
  d.sn_b = s.stride_n * eb;
  d.sl_b = s.stride_l * eb;
  d.cu = s.cu_seqlens;
  d.lengths = s.lengths;
  d.mask = s.mask;
  d.msn = s.mask_stride_n;
  d.msl = s.mask_stride_l;
  d.ts = tensor_scale(s) ? nullptr : s.token_scale;
  d.tsn = s.scale_stride_n;
  d.tsl = s.scale_stride_l;
  d.n = s.n;
  d.L = s.len;
  d.dim = s.dim;
  return d;
}

int check_seqs(const lik_seqs_t* s) {
  if (!s || s->n < 0 || s->len < 0 || s->dim <= 0) return LIK_ERR_INVALID;
  if (s->dtype < LIK_BF16 || s->dtype > LIK_FP8_E4M3) return LIK_ERR_INVALID;
  if (s->n > 0 && s->len > 0 && !s->data) return LIK_ERR_INVALID;
  const int eb = elem_bytes(s->dtype);
  if ((s->dim * eb) % 16 != 0) return LIK_ERR_UNSUPPORTED;
  if (((uintptr_t)s->data) % 16 != 0) return LIK_ERR_UNSUPPORTED;
  if ((s->stride_l * eb) % 16 != 0) return LIK_ERR_UNSUPPORTED;
  if (!s->cu_seqlens && (s->stride_n * eb) % 16 != 0) return LIK_ERR_UNSUPPORTED;
  if (s->cu_seqlens && (s->mask || s->lengths)) return LIK_ERR_INVALID;
  if (s->token_scale && s->dtype != LIK_FP8_E4M3) return LIK_ERR_INVALID;
  // the tile loads address one sequence with 32-bit byte offsets
  if (s->len > 0 && ((s->len - 1) * s->stride_l + s->dim) * (int64_t)eb >= (int64_t)1 << 32) return LIK_ERR_UNSUPPORTED;
  return LIK_OK;
}


// Choose the column block, Lq chunking and grouping for `nq` queries of
// (max) length `lq`. `one_query_per_group` is true when each query owns its
// documents (KD / pairs).
int make_plan(int dt, int dim, int64_t nq, int64_t lq, bool one_query_per_group, Plan& pl, int min_w = 1,
              bool prefer_two_wg = false, const lik_launch_opts_t* opts = nullptr) {
  pl.dpad = pick_dpad(dt, dim);
  if (pl.dpad < 0) return LIK_ERR_UNSUPPORTED;
  const int nsmax = max_nsub(dt, pl.dpad);
  // wide rows: a one-wave workgroup would stage 32+ chunks per thread
  if (pl.dpad >= 256 && min_w < 4) min_w = 4;
  if (lq < 1) lq = 1;
  const int64_t need = one_query_per_group ? lq : nq * lq;
  int best = -1;
  for (int i = 0; i < kNumCfgs; ++i) {
    if (kCfgs[i].NSUB > nsmax) continue;
    if (kCfgs[i].W == 8 && kCfgs[i].NSUB == 4 && dt != LIK_FP8_E4M3) continue;
    if (kCfgs[i].W < min_w) continue;
    // two waves per SIMD (W = 8) leave about 64 VGPRs for query fragments
    if (kCfgs[i].W == 8 && kCfgs[i].NSUB * bfrag_regs(dt, pl.dpad) > 64) continue;
    if (best >= 0 && kCfgs[i].W * kCfgs[i].NSUB <= kCfgs[best].W * kCfgs[best].NSUB) continue;
    best = i;
    if ((int64_t)kCfgs[i].W * kCfgs[i].NSUB * 32 >= need) break;
  }
  if (best < 0) return LIK_ERR_UNSUPPORTED;
  pl.W = kCfgs[best].W;
  pl.NSUB = kCfgs[best].NSUB;
  // Dense bf16 / fp16 scoring: the equally wide 4 x 4 block runs two
  // workgroups per CU (the kernel caps it at 256 registers), which measures
  // faster than one 8-wave workgroup.
  if (prefer_two_wg && pl.W == 8 && pl.NSUB == 2 && nsmax >= 4 && min_w <= 4 && (dt == LIK_BF16 || dt == LIK_F16)) {
    pl.W = 4;
    pl.NSUB = 4;
  }
  // fp8: 4 x 4 at two workgroups per CU beats the one-workgroup 8 x 4, and
  // 4 x 6 (768 columns) beats 4 x 4 by 30% once the call fills a group
  if (prefer_two_wg && pl.W == 8 && pl.NSUB == 4 && min_w <= 4 && dt == LIK_FP8_E4M3) {
    pl.W = 4;
    pl.NSUB = 4;
    if (pl.dpad <= 128 && !one_query_per_group && need >= 4 * 6 * 32) pl.NSUB = 6;
  }
  // a caller-forced column block (lik_launch_opts_t), when this call can use it
  if (opts && opts->col_waves > 0 && opts->col_blocks > 0) {
    const int w = opts->col_waves, ns = opts->col_blocks;
    const bool std_ok = (w == 1 || w == 4 || w == 8) && (ns == 1 || ns == 2 || ns == 4) && ns <= nsmax &&
                        w >= min_w && !(w == 8 && ns * bfrag_regs(dt, pl.dpad) > 64) &&
                        !(w == 8 && ns == 4 && dt != LIK_FP8_E4M3);
    const bool fp8_wide = w == 4 && ns == 6 && dt == LIK_FP8_E4M3 && pl.dpad <= 128 && prefer_two_wg;
    if (std_ok || fp8_wide) {
      pl.W = w;
      pl.NSUB = ns;
    }
  }
  const int cols = pl.W * pl.NSUB * 32;
  if (lq <= cols) {
    pl.nc = 1;
    pl.LU = (int)lq;
    pl.QPG = one_query_per_group ? 1 : cols / (int)lq;
  } else {
    // Split each query into nc chunks; pick the chunking that wastes the
    // fewest columns (MaxSim is a sum over query tokens, so chunks add up).
    double best_eff = -1.0;
    for (int nc = (int)((lq + cols - 1) / cols); nc <= (int)((lq + cols - 1) / cols) + 8; ++nc) {
      const int lu = (int)((lq + nc - 1) / nc);
      const int qpg = one_query_per_group ? 1 : cols / lu;
      const double eff = (double)qpg * lu / cols;
      if (eff > best_eff + 1e-9) {
        best_eff = eff;
        pl.nc = nc;
        pl.LU = lu;
        pl.QPG = qpg;
      }
      if (one_query_per_group) break;
    }
  }
  pl.nunits = nq * pl.nc;
  pl.ngroups = one_query_per_group ? pl.nunits : (pl.nunits + pl.QPG - 1) / pl.QPG;
  return LIK_OK;
}

// Docs per workgroup: aim for >= ~2048 workgroups so 256 CUs see several
// waves of work, but keep at least a few docs per workgroup to amortise the
// query-block load.
// Docs per workgroup. dpad > 0: a dense MaxSim launch of that row width
// (PLAID tiles pass 0: their workgroups are latency-bound, more of them help).
int pick_R(int64_t ngroups, int64_t ndocs, int dpad, const lik_launch_opts_t* opts = nullptr) {
  const int64_t target = 2048;
  int64_t R = (ndocs * ngroups) / target;
  if (ngroups == 1 && dpad > 0) {
    // One query block (a single short query): the launch streams the docs
    // once and every workgroup pays its prologue and pipeline fill. Fewer,
    // longer workgroups win until the grid no longer fills the chip; these
    // workgroup counts measured best on one MI355X for 1k..20k docs of 200 to
    // 300 tokens (d 512: 250, one workgroup per CU; d 128: about 625).
    const int64_t wgs = dpad >= 512 ? 250 : dpad >= 256 ? 750 : dpad >= 128 ? 625 : 1250;
    const int64_t r1 = (ndocs + wgs - 1) / wgs;
    if (r1 > R) R = r1;
  }
  if (opts && opts->docs_per_wg > 0) R = opts->docs_per_wg;  // caller-forced (lik_launch_opts_t)
  if (R < 1) R = 1;
  if (R > ndocs) R = ndocs > 0 ? ndocs : 1;
  if (R > 512) R = 512;  // per-doc metadata of a workgroup lives in LDS (kRMax)
  return (int)R;
}

int launch_dense(int dt, const Plan& pl, const Params& p, int64_t nb, hipStream_t s) {
  if (p.amax) {
    if (q1_eligible(dt, pl, p)) return launch_q1(dt, pl, p, s);
    switch (dt) {
      case LIK_BF16: return launch_dense_train_bf16(pl, p, nb, s);
      case LIK_F16: return launch_dense_train_f16(pl, p, nb, s);
      case LIK_F32: return launch_dense_train_f32(pl, p, nb, s);
      default: return LIK_ERR_UNSUPPORTED;
    }
  }
  if (q1_eligible(dt, pl, p)) return launch_q1(dt, pl, p, s);
  switch (dt) {
    case LIK_BF16: return launch_dense_bf16(pl, p, nb, s);
    case LIK_F16: return launch_dense_f16(pl, p, nb, s);
    case LIK_F32: return launch_dense_f32(pl, p, nb, s);
    case LIK_FP8_E4M3: return launch_dense_fp8(pl, p, nb, s);
    default: return LIK_ERR_UNSUPPORTED;
  }
}

int launch_plaid(int dt, int cd, const Plan& pl, const Params& p, int64_t nb, hipStream_t s) {
  if (dt == LIK_BF16) return launch_plaid_bf16(cd, pl, p, nb, s);
  if (dt == LIK_F16) return launch_plaid_f16(cd, pl, p, nb, s);
  return LIK_ERR_UNSUPPORTED;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Params::normalize bits from the API flags: bit 0 queries, bit 1 docs.
int norm_bits(uint32_t flags) {
  return ((flags & (LIK_NORMALIZE | LIK_NORMALIZE_Q)) ? 1 : 0) | ((flags & (LIK_NORMALIZE | LIK_NORMALIZE_D)) ? 2 : 0);
}

// Times the call's main tile-kernel launches with the caller's HIP events
// (lik_launch_opts_t::timing_start / timing_stop), when both are given.
template <typename F>
int timed_launch(hipStream_t s, const lik_launch_opts_t* opts, F&& launch) {
  TimingScope ts(opts);
  const int rc = launch();
  const int rc2 = ts.close(s);
  return rc != LIK_OK ? rc : rc2;
}

struct WsLayout {
  size_t extent_off = 0, holes_off = 0, tbits_off = 0, part_off = 0, dnorm_off = 0, total = 0;
  bool need_extent = false, need_part = false, need_dnorm = false;
  int64_t dnorm_docs = 0;  // docs per pre-normalised slice
};

// Largest pre-normalised doc copy a call keeps in its workspace: docs are
// normalised and scored in slices of at most this many bytes, so the
// workspace of a large corpus stays bounded (a slice of 512 MiB holds 2M
// bf16 rows of d = 128 and keeps the tile kernel's grid full).
constexpr size_t kPrenormCap = (size_t)512 << 20;

// Doc tokens are normalised once, ahead of the tile kernel, when several
// workgroups would each normalise every doc tile (cross-product scoring with
// more than one query group, padded bf16 / fp16 docs; scoring or the training
// forward alike, the rows are bitwise the kernel's own): the kernel then only
// normalises its query block. `allow` = false keeps the doc normalise in the
// tile kernel (callers without room for the normalised copy).
bool prenorm_docs(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags, const Plan& pl, bool allow) {
  return allow && (norm_bits(flags) & 2) && !(flags & LIK_KD_LAYOUT) && !D->cu_seqlens && pl.ngroups > 1 &&
         (Q->dtype == LIK_BF16 || Q->dtype == LIK_F16) && D->len > 0;
}

// The plan of a scoring call: the two-workgroup 4 x 4 block is preferred when
// the tile loop does no doc-side work (no doc normalise left in the kernel,
// no argmax, no token scales).
int plan_call(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags, bool argmax, Plan& pl, bool& prenorm,
              const lik_launch_opts_t* opts, bool allow_prenorm = true) {
  const bool kd = (flags & LIK_KD_LAYOUT) != 0;
  const int min_w = ((norm_bits(flags) & 2) || argmax) ? 4 : 1;
  const bool plain = !argmax && !row_scale(Q) && !row_scale(D);
  int rc = make_plan(Q->dtype, Q->dim, Q->n, Q->len, kd, pl, min_w, plain, opts);
  if (rc != LIK_OK) return rc;
  prenorm = prenorm_docs(Q, D, flags, pl, allow_prenorm);
  if ((norm_bits(flags) & 2) && !prenorm && plain)  // docs normalised in the kernel: no 4 x 4 preference
    rc = make_plan(Q->dtype, Q->dim, Q->n, Q->len, kd, pl, min_w, false, opts);
  return rc;
}

WsLayout ws_layout(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags, const Plan& pl, bool prenorm) {
  WsLayout w;
  size_t off = 0;
  if (prenorm) {
    const size_t row_doc = (size_t)D->len * (size_t)D->dim * 2;
    int64_t per = (int64_t)(kPrenormCap / row_doc);
    if (per < 1) per = 1;
    w.dnorm_docs = per < D->n ? per : D->n;
    w.need_dnorm = true;
    w.dnorm_off = off;
    off = align256(off + (size_t)w.dnorm_docs * row_doc);
  }
  if (D->mask) {
    w.need_extent = true;
    w.extent_off = off;
    off = align256(off + sizeof(int32_t) * (size_t)D->n);
    w.holes_off = off;
    off = align256(off + (size_t)D->n);
    w.tbits_off = off;
    off = align256(off + sizeof(uint32_t) * (size_t)D->n * (size_t)((D->len + 31) / 32));
  }
  if (pl.nc > 1) {
    const bool kd = (flags & LIK_KD_LAYOUT) != 0;
    const int64_t ndpg = kd ? (Q->n > 0 ? D->n / Q->n : 0) : D->n;
    w.need_part = true;
    w.part_off = off;
    off = align256(off + sizeof(float) * (size_t)(pl.nunits * ndpg));
  }
  w.total = off;
  return w;
}

// Normalised copy of docs [j0, j0 + n) of D, contiguous [n, len, dim], in dst.
int launch_norm_rows(const lik_seqs_t* D, int dpad, int64_t j0, int64_t n, char* dst, hipStream_t s) {
  const int eb = elem_bytes(D->dtype);
  const int64_t rows = n * D->len;
  const int lpr = dpad * eb / 16;  // the tile kernel's chunks per row
  const unsigned nblk = (unsigned)((rows * lpr + 255) / 256);
  const int64_t sn = D->stride_n * eb, sl = D->stride_l * eb;
  const char* dx = (const char*)D->data + j0 * sn;
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(nblk), dim3(256), 0, s, dx, sn, sl, n, D->len, D->dim, dst);
    return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
  };
  if (D->dtype == LIK_BF16) {
    if (lpr == 8) return go(norm_rows_kernel<EK_BF16, 8>);
    if (lpr == 16) return go(norm_rows_kernel<EK_BF16, 16>);
    if (lpr == 32) return go(norm_rows_kernel<EK_BF16, 32>);
    return go(norm_rows_kernel<EK_BF16, 64>);
  }
  if (lpr == 8) return go(norm_rows_kernel<EK_F16, 8>);
  if (lpr == 16) return go(norm_rows_kernel<EK_F16, 16>);
  if (lpr == 32) return go(norm_rows_kernel<EK_F16, 32>);
  return go(norm_rows_kernel<EK_F16, 64>);
}

int launch_fill_i32(int32_t* a, int64_t n, int32_t v, hipStream_t s) {
  if (n <= 0) return LIK_OK;
  hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a, n, v);
  return hipGetLastError() == hipSuccess ? LIK_OK : LIK_ERR_LAUNCH;
}

int maxsim_impl(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags, float out_scale, float* out,
                int64_t out_stride_q, int64_t out_stride_d, int32_t* argmax, void* workspace, size_t workspace_bytes,
                const lik_launch_opts_t* opts, bool allow_prenorm, lik_stream_t stream) {
  int rc;
  if ((rc = check_seqs(Q)) != LIK_OK) return rc;
  if ((rc = check_seqs(D)) != LIK_OK) return rc;
  if (Q->dtype != D->dtype || Q->dim != D->dim) return LIK_ERR_INVALID;
  if (!out && Q->n > 0 && D->n > 0) return LIK_ERR_INVALID;
  const bool kd = (flags & LIK_KD_LAYOUT) != 0;
  if (kd && (D->cu_seqlens || (Q->n > 0 && D->n % Q->n != 0))) return LIK_ERR_INVALID;
  if (Q->n == 0 || D->n == 0) return LIK_OK;
  hipStream_t s = (hipStream_t)stream;

  // rows wider than any column block (bf16 / fp16 > 512, fp32 > 256): the
  // one-wave-per-pair kernel, no workspace
  if (pick_dpad(Q->dtype, Q->dim) < 0) {
    if (Q->dtype == LIK_FP8_E4M3 || Q->token_scale || D->token_scale) return LIK_ERR_UNSUPPORTED;
    Params p{};
    p.q = to_dev(*Q);
    p.d = to_dev(*D);
    p.normalize = norm_bits(flags);
    p.out_scale = out_scale;
    p.out = out;
    p.osq = out_stride_q;
    p.osd = out_stride_d;
    p.kd_K = kd ? D->n / Q->n : 0;
    p.ndocs_pg = kd ? p.kd_K : D->n;
    if (argmax) {
      if ((rc = launch_fill_i32(argmax, Q->n * p.ndocs_pg * Q->len, -1, s)) != LIK_OK) return rc;
      p.amax = argmax;
      p.amax_ld = Q->len;
      p.amax_qs = p.ndocs_pg;
    }
    return timed_launch(s, opts, [&] { return launch_maxsim_wide(Q->dtype, p, s); });
  }

  // doc-side normalise (or the argmax epilogue) adds per-tile VALU work: the
  // plan spreads it over at least 4 waves, or the docs are normalised once
  // ahead of the tile kernel
  Plan pl;
  bool prenorm = false;
  if ((rc = plan_call(Q, D, flags, argmax != nullptr, pl, prenorm, opts, allow_prenorm)) != LIK_OK) return rc;
  const WsLayout wl = ws_layout(Q, D, flags, pl, prenorm);
  if (wl.total > 0 && (!workspace || workspace_bytes < wl.total)) return LIK_ERR_WORKSPACE;

  Params p{};
  p.q = to_dev(*Q);
  p.d = to_dev(*D);
  p.scale_q = tensor_scale(*Q) ? Q->token_scale : nullptr;
  p.scale_d = tensor_scale(*D) ? D->token_scale : nullptr;
  p.normalize = norm_bits(flags);
  p.forced_w = (opts && opts->col_waves > 0 && opts->col_blocks > 0) ? opts->col_waves : 0;
  char* ws = (char*)workspace;
  p.out_scale = out_scale;
  p.nunits = pl.nunits;
  p.nc = pl.nc;
  p.LU = pl.LU;
  p.QPG = pl.QPG;
  p.ngroups = pl.ngroups;
  p.kd_K = kd ? D->n / Q->n : 0;
  p.ndocs_pg = kd ? p.kd_K : D->n;
  if (argmax) {
    // entries no doc-end reaches (empty docs) stay -1
    if ((rc = launch_fill_i32(argmax, Q->n * p.ndocs_pg * Q->len, -1, s)) != LIK_OK) return rc;
    p.amax = argmax;
    p.amax_ld = Q->len;
    p.amax_qs = p.ndocs_pg;
  }

  if (wl.need_extent) {
    p.extent = (const int32_t*)(ws + wl.extent_off);
    p.holes = (const uint8_t*)(ws + wl.holes_off);
    p.tbits = (const uint32_t*)(ws + wl.tbits_off);
    p.tbits_sn = (D->len + 31) / 32;
    const int64_t mend = (D->n - 1) * D->mask_stride_n + D->len;  // one past the mask's last byte
    if (D->mask_stride_l == 1 && D->mask_stride_n >= 0 && D->mask_stride_n % 4 == 0 &&
        (uintptr_t)D->mask % 4 == 0 && D->len <= 1024 && mend < 0x7fffffffLL)
      hipLaunchKernelGGL(doc_extent_w4_kernel, dim3((unsigned)((D->n + 15) / 16)), dim3(256), 0, s, D->mask,
                         D->mask_stride_n, (uint32_t)mend, D->n, (int)D->len, D->lengths,
                         (int32_t*)(ws + wl.extent_off), (uint8_t*)(ws + wl.holes_off),
                         (uint32_t*)(ws + wl.tbits_off), (int)p.tbits_sn);
    else
      hipLaunchKernelGGL(doc_extent_kernel, dim3((unsigned)((D->n + 3) / 4)), dim3(256), 0, s, D->mask,
                         D->mask_stride_n, D->mask_stride_l, D->n, D->len, D->lengths,
                         (int32_t*)(ws + wl.extent_off), (uint8_t*)(ws + wl.holes_off),
                         (uint32_t*)(ws + wl.tbits_off), p.tbits_sn);
    if (hipGetLastError() != hipSuccess) return LIK_ERR_LAUNCH;
  }
  if (wl.need_part) {
    p.out = (float*)(ws + wl.part_off);
    p.osq = p.ndocs_pg;
    p.osd = 1;
  } else {
    p.out = out;
    p.osq = out_stride_q;
    p.osd = out_stride_d;
  }

  // Tile-kernel launches over docs [j0, j0 + n): the workgroup grid, and with
  // masks the two-launch split: docs whose kept tokens form a prefix are
  // scored by the mask-free kernel with the extent as length; a second launch
  // of the masked kernel scores only the docs with holes (its other
  // workgroups exit right after reading the doc table).
  auto score_docs = [&](Params ps, int64_t j0, int64_t n) -> int {
    ps.ndocs_pg = n;
    ps.out += j0 * ps.osd;
    if (ps.extent) {
      ps.extent += j0;
      ps.holes += j0;
      ps.tbits += j0 * ps.tbits_sn;
    }
    if (ps.d.mask) ps.d.mask += j0 * ps.d.msn;
    if (ps.d.lengths) ps.d.lengths += j0;
    if (ps.amax) ps.amax += j0 * ps.amax_ld;
    ps.R = pick_R(ps.ngroups, n, pl.dpad, opts);
    ps.NR = (n + ps.R - 1) / ps.R;
    ps.xcd_map = ps.NR >= 8 ? 1 : 0;
    const int64_t nb = ps.xcd_map ? ps.ngroups * ((ps.NR + 7) / 8) * 8 : ps.ngroups * ps.NR;
    if (ps.extent) {
      Params p1 = ps;
      p1.d.mask = nullptr;
      p1.doc_filter = 1;
      int r = launch_dense(Q->dtype, pl, p1, nb, s);
      if (r != LIK_OK) return r;
      ps.doc_filter = 2;
    }
    return launch_dense(Q->dtype, pl, ps, nb, s);
  };

  if (!wl.need_dnorm) {
    TimingScope ts(opts);
    if ((rc = score_docs(p, 0, p.ndocs_pg)) != LIK_OK) return rc;
    if ((rc = ts.close(s)) != LIK_OK) return rc;
  } else {
    // padded cross-product docs, normalised and scored slice by slice through
    // one bounded copy; the tile kernel then normalises only its query block
    char* dn = ws + wl.dnorm_off;
    const int eb = elem_bytes(D->dtype);
    // the events span the slices' tile kernels: from the first one's start to
    // the last one's end (the later slices' normalisation passes included)
    TimingScope ts(opts);
    for (int64_t j0 = 0; j0 < D->n; j0 += wl.dnorm_docs) {
      const int64_t n = D->n - j0 < wl.dnorm_docs ? D->n - j0 : wl.dnorm_docs;
      if ((rc = launch_norm_rows(D, pl.dpad, j0, n, dn, s)) != LIK_OK) return rc;
      Params ps = p;
      ps.d.data = dn;  // the copy holds the slice's docs from its first one
      ps.d.sn_b = D->len * (int64_t)D->dim * eb;
      ps.d.sl_b = (int64_t)D->dim * eb;
      ps.normalize &= 1;
      if ((rc = score_docs(ps, j0, n)) != LIK_OK) return rc;
    }
    if ((rc = ts.close(s)) != LIK_OK) return rc;
  }
  if (wl.need_part) {
    const int64_t tot = Q->n * p.ndocs_pg;
    hipLaunchKernelGGL(unit_sum_kernel, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s,
                       (const float*)(ws + wl.part_off), Q->n, pl.nc, p.ndocs_pg, out, out_stride_q,
                       out_stride_d);
    if (hipGetLastError() != hipSuccess) return LIK_ERR_LAUNCH;
  }
  return LIK_OK;
}

// Pair-list scoring. Queries longer than one column block are scored in
// chunks of query tokens, one launch per chunk, each adding its partial sums
// to out in chunk order; rows wider than the tile kernel take the
// one-wave-per-pair kernel.
int pairs_impl(const lik_seqs_t* Q, const lik_seqs_t* D, const int32_t* pair_q, const int32_t* pair_d,
               int64_t num_pairs, uint32_t flags, float* out, int32_t* argmax, lik_stream_t stream) {
  int rc;
  if ((rc = check_seqs(Q)) != LIK_OK) return rc;
  if ((rc = check_seqs(D)) != LIK_OK) return rc;
  if (Q->dtype != D->dtype || Q->dim != D->dim) return LIK_ERR_INVALID;
  if (num_pairs < 0 || (num_pairs > 0 && (!pair_q || !pair_d || !out))) return LIK_ERR_INVALID;
  if (D->mask || (flags & LIK_KD_LAYOUT)) return LIK_ERR_INVALID;
  if (num_pairs == 0) return LIK_OK;
  hipStream_t s = (hipStream_t)stream;
  if (argmax && (Q->dtype == LIK_FP8_E4M3 || Q->token_scale || D->token_scale)) return LIK_ERR_UNSUPPORTED;
  Params p{};
  if (argmax) {
    // pairs with no winner stay -1
    if ((rc = launch_fill_i32(argmax, num_pairs * Q->len, -1, s)) != LIK_OK) return rc;
    p.amax = argmax;
    p.amax_ld = Q->len;
    p.amax_qs = 1;
  }
  p.q = to_dev(*Q);
  p.d = to_dev(*D);
  p.scale_q = tensor_scale(*Q) ? Q->token_scale : nullptr;
  p.scale_d = tensor_scale(*D) ? D->token_scale : nullptr;
  p.normalize = norm_bits(flags);
  p.out_scale = 1.f;
  p.pair_q = pair_q;
  p.pair_d = pair_d;
  p.out = out;
  if (pick_dpad(Q->dtype, Q->dim) < 0) {
    if (Q->dtype == LIK_FP8_E4M3 || Q->token_scale || D->token_scale) return LIK_ERR_UNSUPPORTED;
    p.ndocs_pg = 1;
    p.nunits = num_pairs;
    p.osq = 1;
    return launch_maxsim_wide(Q->dtype, p, s);
  }
  Plan pl;
  if ((rc = make_plan(Q->dtype, Q->dim, 1, Q->len, true, pl, argmax ? 4 : 1)) != LIK_OK) return rc;
  p.nunits = num_pairs;
  p.nc = 1;
  p.LU = pl.LU;
  p.QPG = 1;
  p.ngroups = num_pairs;
  p.ndocs_pg = 1;
  p.R = 1;
  p.NR = 1;
  p.xcd_map = 0;
  p.osq = 1;
  p.osd = 0;
  for (int c = 0; c < pl.nc; ++c) {
    p.q_tok0 = (int64_t)c * pl.LU;
    p.accumulate = c > 0;
    if ((rc = launch_dense(Q->dtype, pl, p, num_pairs, s)) != LIK_OK) return rc;
  }
  return LIK_OK;
}

// ---------------------------------------------------------------------------
// Library-owned scratch for lik_maxsim_noalloc: one fixed array per device,
// held until the process ends. Host code never uses the symbol itself (its
// host-side name is not a device address): the array's device address is
// looked up once per device with hipGetSymbolAddress and only that pointer is
// handed to kernels.
constexpr size_t kScratchBytes = LIK_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::once_flag g_scratch_once[kMaxDevices];
void* g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];

// Device address of this device's scratch array (set up on the first call
// that runs on the device, with that device current), or null on failure.
void* device_scratch(hipStream_t s) {
  int dev = 0;
  if (s) {
    hipDevice_t sd;
    if (hipStreamGetDevice(s, &sd) != hipSuccess) return nullptr;
    dev = (int)sd;
  } else if (hipGetDevice(&dev) != hipSuccess) {
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) return nullptr;
  std::call_once(g_scratch_once[dev], [dev] {
    int cur = 0;
    g_scratch_err[dev] = hipGetDevice(&cur);
    if (g_scratch_err[dev] != hipSuccess) return;
    if (cur != dev && (g_scratch_err[dev] = hipSetDevice(dev)) != hipSuccess) return;
    void* ptr = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = g_scratch_err[dev] == hipSuccess ? ptr : nullptr;
    if (cur != dev) (void)hipSetDevice(cur);
  });
  return g_scratch_ptr[dev];
}

}  // namespace


extern "C" {

const char* lik_version(void) { return "lik-hip 0.1.0 gfx950"; }

size_t lik_maxsim_workspace_size_ex(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags,
                                    const lik_launch_opts_t* opts) {
  if (check_seqs(Q) != LIK_OK || check_seqs(D) != LIK_OK) return 0;
  // the same size serves the scoring call and the training forward
  size_t total = 0;
  for (bool argmax : {false, true}) {
    Plan pl;
    bool prenorm = false;
    if (plan_call(Q, D, flags, argmax, pl, prenorm, opts) != LIK_OK) return 0;
    const size_t t = ws_layout(Q, D, flags, pl, prenorm).total;
    total = t > total ? t : total;
  }
  return total;
}

size_t lik_maxsim_workspace_size(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags) {
  return lik_maxsim_workspace_size_ex(Q, D, flags, nullptr);
}

int lik_maxsim(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags, float out_scale, float* out,
               int64_t out_stride_q, int64_t out_stride_d, void* workspace, size_t workspace_bytes,
               lik_stream_t stream) {
  return maxsim_impl(Q, D, flags, out_scale, out, out_stride_q, out_stride_d, nullptr, workspace, workspace_bytes,
                     nullptr, true, stream);
}

int lik_maxsim_ex(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags, float out_scale, float* out,
                  int64_t out_stride_q, int64_t out_stride_d, void* workspace, size_t workspace_bytes,
                  const lik_launch_opts_t* opts, lik_stream_t stream) {
  return maxsim_impl(Q, D, flags, out_scale, out, out_stride_q, out_stride_d, nullptr, workspace, workspace_bytes,
                     opts, true, stream);
}

int lik_maxsim_noalloc(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags, float out_scale, float* out,
                       int64_t out_stride_q, int64_t out_stride_d, lik_stream_t stream) {
  size_t need = 0;
  {
    // the scratch layout this call needs (doc normalise stays in the kernel)
    int rc;
    if ((rc = check_seqs(Q)) != LIK_OK) return rc;
    if ((rc = check_seqs(D)) != LIK_OK) return rc;
    if (Q->n > 0 && D->n > 0 && pick_dpad(Q->dtype, Q->dim) >= 0) {
      Plan pl;
      bool prenorm = false;
      if ((rc = plan_call(Q, D, flags, false, pl, prenorm, nullptr, false)) != LIK_OK) return rc;
      need = ws_layout(Q, D, flags, pl, prenorm).total;
    }
  }
  if (need > kScratchBytes) return LIK_ERR_WORKSPACE;
  void* ws = nullptr;
  if (need > 0 && !(ws = device_scratch((hipStream_t)stream))) return LIK_ERR_LAUNCH;
  return maxsim_impl(Q, D, flags, out_scale, out, out_stride_q, out_stride_d, nullptr, ws, kScratchBytes, nullptr,
                     false, stream);
}

int lik_maxsim_argmax(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags, float* out, int64_t out_stride_q,
                      int64_t out_stride_d, int32_t* argmax, void* workspace, size_t workspace_bytes,
                      lik_stream_t stream) {
  if (!argmax && Q && D && Q->n > 0 && D->n > 0) return LIK_ERR_INVALID;
  if (Q && (Q->dtype == LIK_FP8_E4M3 || Q->token_scale || (D && D->token_scale))) return LIK_ERR_UNSUPPORTED;
  return maxsim_impl(Q, D, flags, 1.0f, out, out_stride_q, out_stride_d, argmax, workspace, workspace_bytes, nullptr,
                     true, stream);
}

int lik_maxsim_pairs(const lik_seqs_t* Q, const lik_seqs_t* D, const int32_t* pair_q, const int32_t* pair_d,
                     int64_t num_pairs, uint32_t flags, float* out, lik_stream_t stream) {
  return pairs_impl(Q, D, pair_q, pair_d, num_pairs, flags, out, nullptr, stream);
}

int lik_maxsim_pairs_argmax(const lik_seqs_t* Q, const lik_seqs_t* D, const int32_t* pair_q, const int32_t* pair_d,
                            int64_t num_pairs, uint32_t flags, float* out, int32_t* argmax, lik_stream_t stream) {
  if (num_pairs > 0 && !argmax) return LIK_ERR_INVALID;
  return pairs_impl(Q, D, pair_q, pair_d, num_pairs, flags, out, argmax, stream);
}

int lik_plaid_maxsim(const lik_seqs_t* Q, const lik_plaid_docs_t* docs, uint32_t flags, float* out,
                     int64_t out_stride_q, int64_t out_stride_d, lik_stream_t stream) {
  return lik_plaid_maxsim_ex(Q, docs, flags, out, out_stride_q, out_stride_d, nullptr, stream);
}

int lik_plaid_maxsim_ex(const lik_seqs_t* Q, const lik_plaid_docs_t* docs, uint32_t flags, float* out,
                        int64_t out_stride_q, int64_t out_stride_d, const lik_launch_opts_t* opts,
                        lik_stream_t stream) {
  int rc;
  if ((rc = check_seqs(Q)) != LIK_OK) return rc;
  if (!docs || docs->n < 0) return LIK_ERR_INVALID;
  if (Q->dtype != LIK_BF16 && Q->dtype != LIK_F16) return LIK_ERR_UNSUPPORTED;
  if (docs->nbits != 2 && docs->nbits != 4 && docs->nbits != 8) return LIK_ERR_INVALID;
  if (docs->dim != Q->dim || Q->dim % 8 != 0) return LIK_ERR_INVALID;
  if (docs->n_buckets < 1 || docs->n_buckets > 256 || !docs->bucket_weights) return LIK_ERR_INVALID;
  if (!docs->cu_seqlens && !docs->lengths) return LIK_ERR_INVALID;
  if (docs->centroid_dtype != LIK_BF16 && docs->centroid_dtype != LIK_F16 && docs->centroid_dtype != LIK_F32)
    return LIK_ERR_UNSUPPORTED;
  if ((flags & LIK_KD_LAYOUT) || Q->mask || Q->token_scale) return LIK_ERR_INVALID;
  if (Q->n == 0 || docs->n == 0) return LIK_OK;
  if (!out || !docs->codes || !docs->residuals || !docs->centroids || docs->n_centroids < 1)
    return LIK_ERR_INVALID;
  const int ceb = elem_bytes(docs->centroid_dtype);
  if (((uintptr_t)docs->centroids) % 16 != 0 || (docs->cent_stride * ceb) % 16 != 0) return LIK_ERR_UNSUPPORTED;
  if (((uintptr_t)docs->residuals) % 8 != 0 || docs->res_stride_tok % docs->nbits != 0)
    return LIK_ERR_UNSUPPORTED;
  if (docs->res_stride_tok * 8 < (int64_t)docs->dim * docs->nbits) return LIK_ERR_INVALID;
  // centroid rows are gathered with 32-bit byte offsets
  if (docs->n_centroids * docs->cent_stride * ceb >= (int64_t)1 << 32) return LIK_ERR_UNSUPPORTED;

  // A few queries (up to 4 of <= 32 tokens): one wavefront per (query, doc
  // range) decodes straight into its MFMA fragments (the tile kernel is
  // latency-bound here).
  const int sdp = pick_dpad(Q->dtype, Q->dim);
  const int variant = opts ? opts->plaid_variant : 0;
  if (Q->n <= 4 && Q->len >= 1 && Q->len <= 32 && (sdp == 64 || sdp == 128) && docs->res_stride_tok % 4 == 0 &&
      docs->centroid_dtype != LIK_F32 && variant != 3) {
    Params p{};
    p.q = to_dev(*Q);
    p.pl.codes = docs->codes;
    p.pl.res = docs->residuals;
    p.pl.cu = docs->cu_seqlens;
    p.pl.lengths = docs->lengths;
    p.pl.n = docs->n;
    p.pl.L = docs->max_len;
    p.pl.codes_sn = docs->codes_stride_n;
    p.pl.res_st = docs->res_stride_tok;
    p.pl.cent = (const char*)docs->centroids;
    p.pl.cent_sb = docs->cent_stride * ceb;
    p.pl.ncent = docs->n_centroids;
    p.pl.bw = docs->bucket_weights;
    p.pl.nb = docs->n_buckets;
    p.pl.nbits = docs->nbits;
    p.normalize = norm_bits(flags);
    p.out_scale = 1.f;
    p.out = out;
    p.osq = out_stride_q;
    p.osd = out_stride_d;
    p.LU = (int)Q->len;
    // LDS-gather variants need 16-byte aligned residual rows and a residual
    // tile no larger than the padded rows'. Centroids of the query's type take
    // the split form (q.c + q.r, norm from its parts: within bf16 / fp16
    // rounding of the decode route, not bitwise equal to it); others the
    // exact decode. plaid_variant 1 / 2 forces the per-lane / the exact
    // gather variant (tuning and parity aids).
    {
      const int64_t rsb = (int64_t)sdp * docs->nbits / 8, nr = (32 * rsb + 1023) / 1024;
      const bool lds_ok = ((uintptr_t)docs->residuals) % 16 == 0 && docs->res_stride_tok % 16 == 0 &&
                          32 * docs->res_stride_tok <= nr * 1024 &&
                          docs->n_centroids * docs->cent_stride * ceb <= (int64_t)kInvRow;
      const bool same_type = docs->centroid_dtype == Q->dtype;
      p.gather = !lds_ok || variant == 1 ? 0 : (same_type && variant != 2 ? 2 : 1);
    }
    // the split form scores two queries per wavefront (one gather and
    // decode serve both); the other variants one
    const int nsub = (p.gather == 2 && Q->n >= 2) ? 2 : 1;
    p.ngroups = (Q->n + nsub - 1) / nsub;
    // ~16k wavefronts over the corpus, at most 512 docs each
    int64_t R = (docs->n + 16383) / 16384;
    p.R = (int)(R < 1 ? 1 : (R > 512 ? 512 : R));
    p.NR = (docs->n + p.R - 1) / p.R;
    const int ek = Q->dtype == LIK_F16 ? EK_F16 : EK_BF16;
    const int cdk = docs->centroid_dtype == LIK_F32 ? EK_F32 : (docs->centroid_dtype == LIK_F16 ? EK_F16 : EK_BF16);
    hipStream_t s = (hipStream_t)stream;
    return timed_launch(s, opts, [&] { return launch_plaid_stream(ek, cdk, sdp, nsub, p, s); });
  }

  Plan pl;
  // PLAID tiles carry the decode VALU work: at least 4 waves share each tile
  // even when the query block would fit one wave's columns.
  if ((rc = make_plan(Q->dtype, Q->dim, Q->n, Q->len, false, pl, 4, false, opts)) != LIK_OK) return rc;
  if (pl.dpad > 256) return LIK_ERR_UNSUPPORTED;
  if (pl.nc != 1) return LIK_ERR_UNSUPPORTED;  // Lq > 512: chunk on the caller side
  Params p{};
  p.q = to_dev(*Q);
  p.pl.codes = docs->codes;
  p.pl.res = docs->residuals;
  p.pl.cu = docs->cu_seqlens;
  p.pl.lengths = docs->lengths;
  p.pl.n = docs->n;
  p.pl.L = docs->max_len;
  p.pl.codes_sn = docs->codes_stride_n;
  p.pl.res_st = docs->res_stride_tok;
  p.pl.cent = (const char*)docs->centroids;
  p.pl.cent_sb = docs->cent_stride * ceb;
  p.pl.ncent = docs->n_centroids;
  p.pl.bw = docs->bucket_weights;
  p.pl.nb = docs->n_buckets;
  p.pl.nbits = docs->nbits;
  p.normalize = norm_bits(flags);
  p.out_scale = 1.f;
  p.nunits = pl.nunits;
  p.nc = 1;
  p.LU = pl.LU;
  p.QPG = pl.QPG;
  p.ngroups = pl.ngroups;
  p.kd_K = 0;
  p.ndocs_pg = docs->n;
  p.out = out;
  p.osq = out_stride_q;
  p.osd = out_stride_d;
  p.R = pick_R(p.ngroups, p.ndocs_pg, 0, opts);
  p.NR = (p.ndocs_pg + p.R - 1) / p.R;
  p.xcd_map = p.NR >= 8 ? 1 : 0;
  const int64_t nb = p.xcd_map ? p.ngroups * ((p.NR + 7) / 8) * 8 : p.ngroups * p.NR;
  return timed_launch((hipStream_t)stream, opts,
                      [&] { return launch_plaid(Q->dtype, docs->centroid_dtype, pl, p, nb, (hipStream_t)stream); });
}

}  // extern "C"
