// Device-visible parameter block of the MaxSim kernels and host-side launch plan.
#pragma once
#include "lik_common.h"

namespace lik {

struct SeqDev {
  const char* data;
  int64_t sn_b, sl_b;  // byte strides
  const int32_t* cu;
  const int32_t* lengths;
  const int8_t* mask;
  int64_t msn, msl;
  const float* ts;
  int64_t tsn, tsl;
  int64_t n, L;
  int dim;
};

struct PlaidDev {
  const int32_t* codes;
  const uint8_t* res;
  const int32_t* cu;
  const int32_t* lengths;
  int64_t n, L, codes_sn, res_st;
  const char* cent;
  int64_t cent_sb;
  int64_t ncent;
  const float* bw;
  int nb, nbits;
};

struct Params {
  SeqDev q;
  SeqDev d;
  PlaidDev pl;
  const int32_t* extent;  // per-doc valid extent from the mask pre-pass
  const uint8_t* holes;   // per-doc: mask has a False inside [0, extent)
  const uint32_t* tbits;  // per (doc, 32-token tile): row-validity bits of the mask
  int64_t tbits_sn;       // tiles per doc in tbits
  int doc_filter;         // 0: all docs; 1: docs without mask holes; 2: docs with holes
  const int32_t* pair_q;
  const int32_t* pair_d;
  int64_t nunits;  // query units (query x Lq-chunk); pair mode: number of pairs
  int nc;          // Lq chunks per query
  int LU;          // columns per unit
  int QPG;         // units per column group
  int64_t ngroups;
  int64_t ndocs_pg;  // docs per group
  int64_t kd_K;      // KD layout: docs per query (0: cross product)
  int R;             // docs per workgroup
  int64_t NR;        // doc ranges per group
  int xcd_map;
  int gather;     // PLAID stream kernel: LDS-gather variant
  int normalize;  // bit 0: L2-normalise query tokens; bit 1: doc tokens
  float out_scale;
  float* out;
  int64_t osq, osd;
  int32_t* amax;    // training forward: winner doc-token index per (query, doc, query token), or null
  int64_t amax_ld;  // query tokens per (query, doc) row of amax (the padded Lq)
  int64_t amax_qs;  // (query, doc) rows of amax per query (the call's docs per query)
  int64_t q_tok0;   // pair mode: first query token of this launch's query chunk
  int accumulate;   // add the scores to out instead of storing them (query-chunk launches)
  const float* scale_q;  // per-tensor scales in device memory folded into the score scale, or null
  const float* scale_d;
  int forced_w;  // caller-forced column block with this many waves (0: the library's plan)
};

// PLAID gather kernel: byte offset given to a row past the tile end; the
// host routes only centroid tables smaller than this to that kernel
constexpr uint32_t kInvRow = 0xfff00000u;

enum { SRC_DENSE = 0, SRC_PLAID = 1 };

__device__ __forceinline__ int64_t seq_len(const SeqDev& s, int64_t i) {
  if (s.cu) return (int64_t)s.cu[i + 1] - s.cu[i];
  if (s.lengths) {
    const int64_t l = s.lengths[i];
    return l < 0 ? 0 : (l > s.L ? s.L : l);
  }
  return s.L;
}
__device__ __forceinline__ const char* seq_row0(const SeqDev& s, int64_t i) {
  return s.cu ? s.data + (int64_t)s.cu[i] * s.sl_b : s.data + i * s.sn_b;
}

template <int SRC>
__device__ __forceinline__ int64_t doc_len(const Params& p, int64_t j) {
  if (j < 0) return 0;  // out-of-range pair index scores 0
  if constexpr (SRC == SRC_PLAID) {
    if (p.pl.cu) return (int64_t)p.pl.cu[j + 1] - p.pl.cu[j];
    const int64_t l = p.pl.lengths[j];
    return l < 0 ? 0 : (l > p.pl.L ? p.pl.L : l);
  } else {
    if (p.extent) return p.extent[j];
    return seq_len(p.d, j);
  }
}

// Config legality: B-fragment registers per lane must stay <= 128 VGPRs.
template <int EK, int DPAD, int NSUB>
constexpr bool cfg_ok() {
  using T = KT<EK, DPAD>;
  return T::KSTEPS >= 1 && T::CPR <= 64 &&
         NSUB * T::KSTEPS * T::FRAG_V * 4 * (T::SPLIT ? 2 : 1) <= 128;
}

// Launch plan chosen on the host (see make_plan in lik_maxsim.hip).
struct Plan {
  int W = 0, NSUB = 0, dpad = 0;
  int LU = 0, QPG = 0, nc = 1;
  int64_t nunits = 0, ngroups = 0;
};

// One per translation unit (lik_inst_*.hip): dispatch on dpad / (W, NSUB).
int launch_dense_bf16(const Plan& pl, const Params& p, int64_t nb, hipStream_t s);
// (lik_inst_*_fast.hip route to specialised feature sets, else to *_generic)
int launch_dense_f16(const Plan& pl, const Params& p, int64_t nb, hipStream_t s);
int launch_dense_f32(const Plan& pl, const Params& p, int64_t nb, hipStream_t s);
int launch_dense_fp8(const Plan& pl, const Params& p, int64_t nb, hipStream_t s);
int launch_plaid_bf16(int cd, const Plan& pl, const Params& p, int64_t nb, hipStream_t s);
// One-column-block plans (lik_q1.hip): the streaming kernel when the call
// qualifies (q1_eligible), else the tile kernel.
bool q1_eligible(int dt, const Plan& pl, const Params& p);
int launch_q1(int dt, const Plan& pl, const Params& p, hipStream_t s);
// Few-query PLAID scoring, one wavefront per (query group, doc range): lik_plaid_stream.hip.
int launch_plaid_stream(int ek, int cd, int dpad, int nsub, const Params& p, hipStream_t s);
// rows wider than the tile kernel takes (lik_wide.hip): one wave per (query, doc)
int launch_maxsim_wide(int dtype, const Params& p, hipStream_t s);
// training forward (argmax output), lik_inst_train_*.hip
int launch_dense_train_bf16(const Plan& pl, const Params& p, int64_t nb, hipStream_t s);
int launch_dense_train_f16(const Plan& pl, const Params& p, int64_t nb, hipStream_t s);
int launch_dense_train_f32(const Plan& pl, const Params& p, int64_t nb, hipStream_t s);
int launch_plaid_f16(int cd, const Plan& pl, const Params& p, int64_t nb, hipStream_t s);

}  // namespace lik
