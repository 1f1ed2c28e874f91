// Shared device-side definitions for the gfx950 MaxSim kernels.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "lik.h"

namespace lik {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Timing of a call's main launches with the caller's HIP events
// (lik_launch_opts_t::timing_start / timing_stop). While a TimingScope is open
// on the calling host thread, every launch made through launch_kernel carries
// the events in its own dispatch (hipExtLaunchKernelGGL): the first records
// timing_start when it starts, each records timing_stop when it ends. No
// event packets are queued between launches, so timed calls run back to back
// like untimed ones (separate hipEventRecord packets left gaps of several us
// around each launch, and a power-limited kernel runs faster after a gap).
struct LaunchTiming {
  hipEvent_t start, stop;
  bool start_pending;
};
inline thread_local LaunchTiming* g_launch_timing = nullptr;

template <typename K, typename... A>
inline void launch_kernel(K kern, dim3 grid, dim3 block, uint32_t shmem, hipStream_t s, A... args) {
  if (LaunchTiming* t = g_launch_timing) {
    hipExtLaunchKernelGGL(kern, grid, block, shmem, s, t->start_pending ? t->start : nullptr, t->stop, 0u, args...);
    t->start_pending = false;
  } else {
    hipLaunchKernelGGL(kern, grid, block, shmem, s, args...);
  }
}

class TimingScope {
 public:
  explicit TimingScope(const lik_launch_opts_t* o) {
    if (o && o->timing_start && o->timing_stop) {
      t_ = LaunchTiming{(hipEvent_t)o->timing_start, (hipEvent_t)o->timing_stop, true};
      prev_ = g_launch_timing;
      g_launch_timing = &t_;
      on_ = true;
    }
  }
  TimingScope(const TimingScope&) = delete;
  TimingScope& operator=(const TimingScope&) = delete;
  // Ends the scope. A scope whose call launched nothing records both events
  // here, back to back (zero duration), so the caller can always read them.
  int close(hipStream_t s) {
    if (!on_) return LIK_OK;
    g_launch_timing = prev_;
    on_ = false;
    if (t_.start_pending &&
        (hipEventRecord(t_.start, s) != hipSuccess || hipEventRecord(t_.stop, s) != hipSuccess))
      return LIK_ERR_LAUNCH;
    return LIK_OK;
  }
  ~TimingScope() {
    if (on_) g_launch_timing = prev_;
  }

 private:
  LaunchTiming t_{};
  LaunchTiming* prev_ = nullptr;
  bool on_ = false;
};

// Element kinds of the token embeddings. F32 is computed as three bf16 MFMAs
// (hi*hi + hi*lo + lo*hi; split_hi / split_lo), ~1e-5 relative of exact fp32 MaxSim.
enum { EK_BF16 = 0, EK_F16 = 1, EK_F32 = 2, EK_FP8 = 3 };

// Compile-time layout of one 32-token tile for element kind EK and padded
// embedding dim DPAD. MFMA 32x32xK: the doc tile is the A operand (32 rows =
// doc tokens), the query block is the B operand (32 columns = query tokens).
// Lane l holds row/column l%32; its half h=l/32 covers embedding elements
// [h*DPAD/2, (h+1)*DPAD/2). The same element order is used for A and B, so
// the dot product is over the same dims whatever the hardware k-ordering is.
template <int EK, int DPAD>
struct KT {
  static constexpr int IN_B = EK == EK_F32 ? 4 : (EK == EK_FP8 ? 1 : 2);  // input bytes/elem
  static constexpr int CB = EK == EK_FP8 ? 1 : 2;          // bytes/elem in LDS
  static constexpr bool SPLIT = EK == EK_F32;
  static constexpr int FE = EK == EK_FP8 ? 32 : 8;          // elems per lane per MFMA
  static constexpr int KSTEPS = DPAD / (2 * FE);            // MFMAs per 32x32 tile
  static constexpr int FRAG_B = FE * CB;                    // 16 or 32 bytes
  static constexpr int FRAG_V = FRAG_B / 16;                // u32x4 per fragment
  static constexpr int HALF_B = DPAD * CB / 2;
  static constexpr int ROW_B = DPAD * CB + 16;              // +16 B pad: conflict-free ds_read_b128
  static constexpr int TILE_B = 32 * ROW_B;
  static constexpr int NARR = SPLIT ? 2 : 1;
  static constexpr int CPR = DPAD * IN_B / 16;              // 16-B input chunks per row
  static constexpr int CHUNK_E = 16 / IN_B;                 // elements per input chunk
  static_assert(KSTEPS >= 1, "DPAD too small for element kind");
  static_assert(CPR <= 64, "a row must be reduced within one wavefront");
};

// D = A x B + C for one 32x32 tile step (A, B: this lane's fragments).
template <int EK>
__device__ __forceinline__ f32x16 mfma32(const f32x16& c, const u32x4* a, const u32x4* b) {
  if constexpr (EK == EK_BF16 || EK == EK_F32) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a[0]),
                                                   __builtin_bit_cast(bf16x8, b[0]), c, 0, 0, 0);
  } else if constexpr (EK == EK_F16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a[0]),
                                                  __builtin_bit_cast(f16x8, b[0]), c, 0, 0, 0);
  } else {
    const i32x8 av = __builtin_bit_cast(i32x8, __builtin_shufflevector(a[0], a[1], 0, 1, 2, 3, 4, 5, 6, 7));
    const i32x8 bv = __builtin_bit_cast(i32x8, __builtin_shufflevector(b[0], b[1], 0, 1, 2, 3, 4, 5, 6, 7));
    // cbsz = blgp = 0: both operands OCP fp8 e4m3; E8M0 scale 127 == 1.0.
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, c, 0, 0, 0, 127, 0, 127);
  }
}

// c + a.lo * b.lo + a.hi * b.hi on packed 16-bit pairs, fp32 accumulate.
template <int EK>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  typedef short s16x2 __attribute__((ext_vector_type(2)));
  if constexpr (EK == EK_F16)
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
  else
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(s16x2, a), __builtin_bit_cast(s16x2, b), c, false);
}

__device__ __forceinline__ float bf16lo_to_f32(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi_to_f32(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// Round-to-nearest-even fp32 -> bf16 bits.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// OCP e4m3fn -> fp32 (exact). Used only for the norms of fp8 rows.
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
  const uint32_t s = (b >> 7) & 1u, e = (b >> 3) & 15u, m = b & 7u;
  float v;
  if (e == 0) v = (float)m * 0.001953125f;  // m * 2^-9
  else if (e == 15 && m == 7) v = __builtin_nanf("");
  else v = __uint_as_float(((e + 120u) << 23) | (m << 20));
  return s ? -v : v;
}

// Sum of squares of a 16-byte chunk of elements of kind EK (F32: 4 floats).
template <int EK>
__device__ __forceinline__ float chunk_sumsq(const u32x4& v) {
  float s = 0.f;
  if constexpr (EK == EK_BF16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = bf16lo_to_f32(v[i]), b = bf16hi_to_f32(v[i]);
      s = fmaf(a, a, s);
      s = fmaf(b, b, s);
    }
  } else if constexpr (EK == EK_F16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = f16_to_f32((uint16_t)(v[i] & 0xffffu)), b = f16_to_f32((uint16_t)(v[i] >> 16));
      s = fmaf(a, a, s);
      s = fmaf(b, b, s);
    }
  } else if constexpr (EK == EK_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = __uint_as_float(v[i]);
      s = fmaf(a, a, s);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float a = e4m3_to_f32((v[i] >> (8 * k)) & 0xffu);
        s = fmaf(a, a, s);
      }
    }
  }
  return s;
}

// fp32 -> bf16 hi / lo split for the three-product fp32 MaxSim
// (hi*hi + hi*lo + lo*hi). hi is x truncated toward zero (NaN stays NaN), so
// lo = x - hi (exact in fp32, then rounded to bf16) has the sign of x: for
// an infinite operand a, a*hi_b and a*lo_b are infinities of one sign and
// never add up to inf - inf = NaN where the true product a*b is +-inf. A lo
// that is zero or subnormal becomes the smallest normal bf16 with x's sign
// (an exactly representable b would otherwise give inf * 0 = NaN); for
// finite operands that stand-in moves a product by at most 2^-126 |y|.
// A non-finite x has lo = that stand-in too. Scores are within ~1e-5
// relative of exact fp32 MaxSim on N(0,1) data (measured against fp64).
__device__ __forceinline__ uint32_t split_hi(float x) {
  return x != x ? 0x7fc0u : (__float_as_uint(x) >> 16);
}
__device__ __forceinline__ uint32_t split_lo(uint32_t hbits, float x) {
  const float r = x - __uint_as_float(hbits << 16);
  const uint32_t l = __builtin_isfinite(r) ? f32_to_bf16_bits(r) : 0u;
  return (l & 0x7f80u) ? l : ((hbits & 0x8000u) | 0x0080u);
}

// Split 4 floats into bf16 hi and lo parts (x ~= hi + lo), packed 2 per u32.
__device__ __forceinline__ void split4(const u32x4& v, u32x2& hi, u32x2& lo) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float a = __uint_as_float(v[2 * i]), b = __uint_as_float(v[2 * i + 1]);
    const uint32_t ha = split_hi(a), hb = split_hi(b);
    hi[i] = ha | (hb << 16);
    lo[i] = split_lo(ha, a) | (split_lo(hb, b) << 16);
  }
}

// max(a, b) that propagates NaN (IEEE 754-2019 maximum; v_maximum3_f32 on
// gfx950). Row maxima use it so that a NaN similarity makes the max NaN, which
// the doc-end test then scores as 0, as torch's max does before the
// isfinite -> 0 rule (reference.py:83-85). fmaxf would drop the NaN and
// score the row from its other tokens.
__device__ __forceinline__ float max_nan(float a, float b) { return __builtin_elementwise_maximum(a, b); }

__device__ __forceinline__ float inv_norm(float ss) {
  // F.normalize: x / max(||x||, 1e-12)
  return 1.0f / fmaxf(sqrtf(ss), 1e-12f);
}

}  // namespace lik
