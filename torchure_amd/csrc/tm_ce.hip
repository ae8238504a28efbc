// tm_ce.hip -- gfx950 kernels of the chunked fused linear + cross-entropy.
//
// The reference (torchure/loss/fused_linear_ce.py:31-59) computes, per chunk of rows,
//   logits = h @ W^T (bf16 GEMM), lse = logsumexp(float(logits)), loss = lse - target,
//   grad_logits = bf16(softmax - onehot) on valid rows (0 on ignored rows),
//   grad_h = grad_logits @ W, grad_W += grad_logits^T @ h,
// and scales both grads by grad_out / n_valid in backward (:94-127).
// The GEMMs are plain library GEMMs (hipBLASLt). These kernels do the rest:
//   ce_rows_kernel        one workgroup per row: row max, sum of exp, target logit,
//                         per-row loss, then softmax - onehot written back over the
//                         logits as bf16 (RNE). A row of up to kRegCols vectors per
//                         thread stays in registers (one HBM read, one write); longer
//                         rows use an online (max, sum-of-exp) read, then a second
//                         read for the write pass. exp is the hardware base-2 exp
//                         (full-range exp2f wherever a result would be denormal), and
//                         the bf16 rounding is the hardware RNE convert.
//   ce_loss_kernel        one workgroup: fixed-order sum of the per-row losses and of
//                         the valid-row count -> loss_sum, n_valid, mean loss.
//   ce_scale_kernel       backward: grad_h (bf16) *= bf16(g / n_valid),
//                         grad_W (fp32) *= g / n_valid.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <type_traits>

#include "torchure_amd.h"
#include "tm_internal.h"

#pragma clang fp contract(off)

namespace {

constexpr int kRowThreadsRegs = 1024;   // 16 wave64 per row when the row stays in registers
constexpr int kRowThreadsStream = 256;  // threads per row on the streaming path (longer rows)
constexpr int kStreamUnroll = 4;  // vectors per thread loaded together on the streaming path
constexpr int kRegCols = 20;  // 8-element vectors per thread kept in registers (V <= 163,840)
constexpr int kMaxWaves = (kRowThreadsRegs > kRowThreadsStream ? kRowThreadsRegs : kRowThreadsStream) / 64;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename... A>
int ce_fail(int code, const char* fmt, A... args) {
  return tm_internal_fail(code, fmt, args...);
}

__device__ __forceinline__ float lo16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi16(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ uint32_t rne16(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
  return (f != f) ? 0x7FC0u : r;
}

constexpr float kLog2e = 1.4426950408889634f;

// The exponent (x - c) * log2(e) of exp(x - c). With kFold it is one fma against the
// precomputed cl = c * log2(e); cl carries an absolute rounding error of half an ulp of
// |c| * log2(e), which for |c| <= kFoldMax is at most 3.8e-6 (a relative error below
// 2.6e-6 in the result, far under half a bf16 ulp). Rows with larger |c| take the two-step
// form, exact at x = c and accurate at any magnitude.
constexpr float kFoldMax = 64.0f;

template <bool kFold>
__device__ __forceinline__ float tlog2(float x, float c, float cl) {
  return kFold ? fmaf(x, kLog2e, -cl) : (x - c) * kLog2e;
}

// exp(x - c) through the base-2 exponential: exp2((x - c) * log2(e)), full range
// (denormal results included).
__device__ __forceinline__ float exp_shift(float x, float c) { return exp2f((x - c) * kLog2e); }

// The bare v_exp_f32: identical to exp2f for results >= 2^-126, flushes smaller ones.
__device__ __forceinline__ float exp2_hw(float t) { return __builtin_amdgcn_exp2f(t); }

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two floats -> packed bf16 (round to nearest even) in one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const bf16x2 h = __builtin_convertvector(f32x2{a, b}, bf16x2);
  return __builtin_bit_cast(uint32_t, h);
}

// (max, sum of exp(x - max)) pairs combine associatively.
__device__ __forceinline__ void ms_merge(float& m, float& s, float m2, float s2) {
  if (m2 == -INFINITY) return;
  if (m2 > m) {
    s = s * exp_shift(m, m2) + s2;
    m = m2;
  } else if (m2 == m) {
    s = s + s2;
  } else {
    s = s + s2 * exp_shift(m2, m);
  }
}

__device__ __forceinline__ void ms_add(float& m, float& s, float x) {
  if (x == -INFINITY) return;  // exp(-inf - m) = 0 contributes nothing
  if (x > m) {
    s = s * exp_shift(m, x) + 1.0f;
    m = x;
  } else {
    s = s + exp_shift(x, m);
  }
}

// Block-wide (max, sumexp) in a fixed order; every thread receives the result.
template <int kCeThreads>
__device__ __forceinline__ void block_ms(float& m, float& s) {
  constexpr int kCeWaves = kCeThreads / 64;
  __shared__ float lm[kMaxWaves], ls[kMaxWaves];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float m2 = __shfl_xor(m, off, 64);
    const float s2 = __shfl_xor(s, off, 64);
    ms_merge(m, s, m2, s2);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    lm[wave] = m;
    ls[wave] = s;
  }
  __syncthreads();
  m = lm[0];
  s = ls[0];
  for (int w = 1; w < kCeWaves; ++w) ms_merge(m, s, lm[w], ls[w]);
  __syncthreads();
}

template <int kCeThreads>
__device__ __forceinline__ float block_max(float m) {
  constexpr int kCeWaves = kCeThreads / 64;
  __shared__ float lm[kMaxWaves];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if ((threadIdx.x & 63) == 0) lm[threadIdx.x >> 6] = m;
  __syncthreads();
  m = lm[0];
  for (int w = 1; w < kCeWaves; ++w) m = fmaxf(m, lm[w]);
  __syncthreads();
  return m;
}

// Block-wide max of a and max of b in one reduction (b carries a negated minimum).
template <int kCeThreads>
__device__ __forceinline__ void block_max2(float& a, float& b) {
  constexpr int kCeWaves = kCeThreads / 64;
  __shared__ float la[kMaxWaves], lb[kMaxWaves];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    a = fmaxf(a, __shfl_xor(a, off, 64));
    b = fmaxf(b, __shfl_xor(b, off, 64));
  }
  if ((threadIdx.x & 63) == 0) {
    la[threadIdx.x >> 6] = a;
    lb[threadIdx.x >> 6] = b;
  }
  __syncthreads();
  a = la[0];
  b = lb[0];
  for (int w = 1; w < kCeWaves; ++w) {
    a = fmaxf(a, la[w]);
    b = fmaxf(b, lb[w]);
  }
  __syncthreads();
}

template <int kCeThreads>
__device__ __forceinline__ float block_sum_f(float s) {
  constexpr int kCeWaves = kCeThreads / 64;
  __shared__ float ls[kMaxWaves];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if ((threadIdx.x & 63) == 0) ls[threadIdx.x >> 6] = s;
  __syncthreads();
  s = ls[0];
  for (int w = 1; w < kCeWaves; ++w) s += ls[w];
  __syncthreads();
  return s;
}

// logits: rows x vocab bf16 (row-major, row stride ld elements), overwritten with
// grad_logits (kGrad; without it the logits are only read). labels: int64 per row.
// row_loss: fp32 per row (0 for ignored rows).
template <bool kInRegs, int kCeThreads, bool kGrad>
__global__ __launch_bounds__(kCeThreads) void ce_rows_kernel(uint16_t* __restrict__ logits,
                                                             int64_t ld,
                                                             const int64_t* __restrict__ labels,
                                                             int64_t vocab, int64_t ignore_index,
                                                             float* __restrict__ row_loss) {
  const int64_t r = blockIdx.x;
  uint16_t* row = logits + r * ld;
  const int64_t label = labels[r];
  const bool valid = label != ignore_index;
  const int64_t nvec = vocab >> 3;  // full 8-element vectors (16 B)
  const bool vec = ((reinterpret_cast<uint64_t>(row) & 15u) == 0);
  const int64_t vend = vec ? nvec * 8 : 0;

  u32x4 keep[kInRegs ? kRegCols : 1];
  float lse;
  float row_min = -INFINITY;  // known only on the register path
  if constexpr (kInRegs) {
    // The row stays in registers: max pass, then sum-of-exp pass, no second read.
    float m = -INFINITY;
    float nmin = -INFINITY;  // -(row minimum), reduced with the maximum
    if (vec && nvec > 0) {
      // Every load is issued before any is used (fully unrolled, compile-time indices, so
      // `keep` stays in VGPRs): a load under a per-thread branch next to its use made each
      // of them wait for the one before. A thread past the row's last vector loads that
      // last vector again, a real element of the row, which leaves the max and min as they
      // are; the sum and the stores below skip those slots. The loss-only pass reads the
      // row non-temporally: 3-22% faster than temporal loads from 1024 to 8192 rows of the
      // Qwen3 vocabulary (same bits); the gradient pass, which rewrites the row, measured
      // no better with them at 2048 rows and beyond.
#pragma unroll
      for (int k = 0; k < kRegCols; ++k) {
        const int64_t v = threadIdx.x + static_cast<int64_t>(k) * kCeThreads;
        const u32x4* src = reinterpret_cast<const u32x4*>(row + (v < nvec ? v : nvec - 1) * 8);
        keep[k] = kGrad ? *src : __builtin_nontemporal_load(src);
      }
      __builtin_amdgcn_sched_barrier(0);  // keep the scheduler from starting the max before the last load
#pragma unroll
      for (int k = 0; k < kRegCols; ++k) {
        const u32x4 w = keep[k];
        m = fmaxf(m, fmaxf(fmaxf(fmaxf(lo16(w.x), hi16(w.x)), fmaxf(lo16(w.y), hi16(w.y))),
                           fmaxf(fmaxf(lo16(w.z), hi16(w.z)), fmaxf(lo16(w.w), hi16(w.w)))));
        nmin = fmaxf(nmin, -fminf(fminf(fminf(lo16(w.x), hi16(w.x)), fminf(lo16(w.y), hi16(w.y))),
                                  fminf(fminf(lo16(w.z), hi16(w.z)), fminf(lo16(w.w), hi16(w.w)))));
      }
    }
    for (int64_t i = vend + threadIdx.x; i < vocab; i += kCeThreads) {
      const float x = __uint_as_float(static_cast<uint32_t>(row[i]) << 16);
      m = fmaxf(m, x);
      nmin = fmaxf(nmin, -x);
    }
    block_max2<kCeThreads>(m, nmin);
    row_min = -nmin;
    const float cm = m * kLog2e;
    // terms below 2^-126 (flushed by the bare exp) cannot move a sum that is >= 1
    auto sum_exp = [&](auto fold) {
      constexpr bool F = decltype(fold)::value;
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < kRegCols; ++k) {
        const int64_t v = threadIdx.x + static_cast<int64_t>(k) * kCeThreads;
        if (v < nvec) {
          const u32x4 w = keep[k];
          acc += exp2_hw(tlog2<F>(lo16(w.x), m, cm)) + exp2_hw(tlog2<F>(hi16(w.x), m, cm)) +
                 exp2_hw(tlog2<F>(lo16(w.y), m, cm)) + exp2_hw(tlog2<F>(hi16(w.y), m, cm)) +
                 exp2_hw(tlog2<F>(lo16(w.z), m, cm)) + exp2_hw(tlog2<F>(hi16(w.z), m, cm)) +
                 exp2_hw(tlog2<F>(lo16(w.w), m, cm)) + exp2_hw(tlog2<F>(hi16(w.w), m, cm));
        }
      }
      return acc;
    };
    float s = 0.0f;
    if (vec) s = fabsf(m) <= kFoldMax ? sum_exp(std::true_type{}) : sum_exp(std::false_type{});
    for (int64_t i = vend + threadIdx.x; i < vocab; i += kCeThreads)
      s += exp_shift(__uint_as_float(static_cast<uint32_t>(row[i]) << 16), m);
    s = block_sum_f<kCeThreads>(s);
    lse = m + logf(s);
  } else {
    // Row too long for registers: one online (max, sum-of-exp) read, one write pass.
    float m = -INFINITY, s = 0.0f;
    if (vec) {
      // 8 independent (max, sum) pairs per thread (one per vector lane) for ILP
      float mm[8], ss[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        mm[j] = -INFINITY;
        ss[j] = 0.0f;
      }
      auto add8 = [&](const u32x4 w) {
        ms_add(mm[0], ss[0], lo16(w.x)); ms_add(mm[1], ss[1], hi16(w.x));
        ms_add(mm[2], ss[2], lo16(w.y)); ms_add(mm[3], ss[3], hi16(w.y));
        ms_add(mm[4], ss[4], lo16(w.z)); ms_add(mm[5], ss[5], hi16(w.z));
        ms_add(mm[6], ss[6], lo16(w.w)); ms_add(mm[7], ss[7], hi16(w.w));
      };
      // kStreamUnroll loads in flight before they are used, same element order per lane
      int64_t v = threadIdx.x;
      for (; v + (kStreamUnroll - 1) * kCeThreads < nvec; v += kStreamUnroll * kCeThreads) {
        u32x4 w[kStreamUnroll];
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u)
          w[u] = *reinterpret_cast<const u32x4*>(row + (v + u * kCeThreads) * 8);
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) add8(w[u]);
      }
      for (; v < nvec; v += kCeThreads) add8(*reinterpret_cast<const u32x4*>(row + v * 8));
#pragma unroll
      for (int j = 0; j < 8; ++j) ms_merge(m, s, mm[j], ss[j]);
    }
    for (int64_t i = vend + threadIdx.x; i < vocab; i += kCeThreads)
      ms_add(m, s, __uint_as_float(static_cast<uint32_t>(row[i]) << 16));
    block_ms<kCeThreads>(m, s);
    lse = m + logf(s);
  }

  // every thread has the same lse; the target logit is read before any write
  const float target = (valid && label >= 0 && label < vocab)
                           ? __uint_as_float(static_cast<uint32_t>(row[label]) << 16)
                           : 0.0f;
  __syncthreads();
  // A label outside [0, vocab) that is not ignore_index makes the reference's gather fail
  // (a device-side assert); here the row's loss is NaN, so the mean loss shows it without a
  // host synchronisation. Its gradient row is the plain softmax.
  const bool in_range = label >= 0 && label < vocab;
  if (threadIdx.x == 0) row_loss[r] = !valid ? 0.0f : (in_range ? lse - target : __builtin_nanf(""));
  if constexpr (!kGrad) return;  // loss only: no gradient pass (no barrier follows)

  // grad = exp(x - lse) on valid rows (0 on ignored rows), minus 1 at the label.
  auto g_of = [&](float x, int64_t idx) -> float {
    if (!valid) return 0.0f;
    float p = exp_shift(x, lse);
    if (idx == label) p = p - 1.0f;
    return p;
  };
  const int64_t label_vec = (valid && label >= 0) ? (label >> 3) : -1;
  const float cl = lse * kLog2e;
  const bool fold = fabsf(lse) <= kFoldMax;
  // both exponent forms are monotonic in x, so the smallest exponent of the row is the row
  // minimum's: if it is >= -126 no result of the row is denormal and every vector takes the
  // bare exp (row_min is -inf on the streaming path, which then checks per vector)
  const bool row_fast = (fold ? tlog2<true>(row_min, lse, cl) : tlog2<false>(row_min, lse, cl)) >= -126.0f;
  auto put8 = [&](const u32x4 w, int64_t v, auto fold_tag) {
    constexpr bool F = decltype(fold_tag)::value;
    const int64_t b = v * 8;
    u32x4 o;
    if (!valid) {
      o = u32x4{0u, 0u, 0u, 0u};
    } else {
      float t[8] = {tlog2<F>(lo16(w.x), lse, cl), tlog2<F>(hi16(w.x), lse, cl),
                    tlog2<F>(lo16(w.y), lse, cl), tlog2<F>(hi16(w.y), lse, cl),
                    tlog2<F>(lo16(w.z), lse, cl), tlog2<F>(hi16(w.z), lse, cl),
                    tlog2<F>(lo16(w.w), lse, cl), tlog2<F>(hi16(w.w), lse, cl)};
      float p[8];
      bool fast = row_fast;
      if (!fast) {
        const float tmin = fminf(fminf(fminf(t[0], t[1]), fminf(t[2], t[3])),
                                 fminf(fminf(t[4], t[5]), fminf(t[6], t[7])));
        fast = tmin >= -126.0f;
      }
      if (fast) {
#pragma unroll
        for (int j = 0; j < 8; ++j) p[j] = exp2_hw(t[j]);
      } else {  // some result is a denormal: the full-range exp2
#pragma unroll
        for (int j = 0; j < 8; ++j) p[j] = exp2f(t[j]);
      }
      if (v == label_vec) p[label & 7] = p[label & 7] - 1.0f;
      o.x = pack_bf16x2(p[0], p[1]);
      o.y = pack_bf16x2(p[2], p[3]);
      o.z = pack_bf16x2(p[4], p[5]);
      o.w = pack_bf16x2(p[6], p[7]);
    }
    // non-temporal: the GEMMs that read grad_logits next find none of it in cache anyway
    // (0.3-2.5 GB); 0-7% faster than temporal stores from 8192 down to 1024 rows
    __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(row + b));
  };
  auto write_row = [&](auto fold_tag) {
    if constexpr (kInRegs) {
#pragma unroll
      for (int k = 0; k < kRegCols; ++k) {
        const int64_t v = threadIdx.x + static_cast<int64_t>(k) * kCeThreads;
        if (v < nvec) put8(keep[k], v, fold_tag);
      }
    } else {
      int64_t v = threadIdx.x;
      for (; v + (kStreamUnroll - 1) * kCeThreads < nvec; v += kStreamUnroll * kCeThreads) {
        u32x4 w[kStreamUnroll];
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u)
          w[u] = *reinterpret_cast<const u32x4*>(row + (v + u * kCeThreads) * 8);
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) put8(w[u], v + u * kCeThreads, fold_tag);
      }
      for (; v < nvec; v += kCeThreads) put8(*reinterpret_cast<const u32x4*>(row + v * 8), v, fold_tag);
    }
  };
  if (vec) {
    if (fold) write_row(std::true_type{});
    else write_row(std::false_type{});
  }
  for (int64_t i = vend + threadIdx.x; i < vocab; i += kCeThreads)
    row[i] = static_cast<uint16_t>(rne16(g_of(__uint_as_float(static_cast<uint32_t>(row[i]) << 16), i)));
}

// (max, sum of exp(x - max)) with the full-precision expf, for fp32 outputs.
__device__ __forceinline__ void ms_merge_f(float& m, float& s, float m2, float s2) {
  if (m2 == -INFINITY) return;
  if (m2 > m) {
    s = s * expf(m - m2) + s2;
    m = m2;
  } else if (m2 == m) {
    s = s + s2;
  } else {
    s = s + s2 * expf(m2 - m);
  }
}

__device__ __forceinline__ void ms_add_f(float& m, float& s, float x) {
  if (x == -INFINITY) return;
  if (x > m) {
    s = s * expf(m - x) + 1.0f;
    m = x;
  } else {
    s = s + expf(x - m);
  }
}

// Block-wide (max, sumexp) of 256-thread workgroups, fixed order, full-precision exp.
__device__ __forceinline__ void block_ms_f(float& m, float& s) {
  __shared__ float lm[4], ls[4];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float m2 = __shfl_xor(m, off, 64);
    const float s2 = __shfl_xor(s, off, 64);
    ms_merge_f(m, s, m2, s2);
  }
  if ((threadIdx.x & 63) == 0) {
    lm[threadIdx.x >> 6] = m;
    ls[threadIdx.x >> 6] = s;
  }
  __syncthreads();
  m = lm[0];
  s = ls[0];
  for (int w = 1; w < 4; ++w) ms_merge_f(m, s, lm[w], ls[w]);
  __syncthreads();
}

// fp32 logits: hidden states and weight in fp32 outside autocast, where the reference's
// products are fp32 GEMMs (fused_linear_ce.py:38,52,57 with w = weight.to(hidden.dtype) at
// :65) and its chunk math runs on fp32 logits (:39-51). One 256-thread workgroup per row and
// two reads of it: an online (max, sum of exp) pass, lse = max + log(sum); then (kGrad) the
// gradient in place, exp(x - lse) on valid rows (0 on ignored rows) minus 1 at the label,
// with the reference's rounding steps: the fp32 difference x - lse, then a full-precision exp.
template <bool kGrad>
__global__ __launch_bounds__(256) void ce_rows_f32_kernel(float* __restrict__ logits, int64_t ld,
                                                          const int64_t* __restrict__ labels, int64_t vocab,
                                                          int64_t ignore_index, float* __restrict__ row_loss) {
  const int64_t r = blockIdx.x;
  float* row = logits + r * ld;
  const int64_t label = labels[r];
  const bool valid = label != ignore_index;
  const int64_t nvec = vocab >> 2;  // full 4-element vectors (16 B)
  const bool vec = ((reinterpret_cast<uint64_t>(row) & 15u) == 0);
  const int64_t vend = vec ? nvec * 4 : 0;
  float m = -INFINITY, s = 0.0f;
  if (vec) {
    float mm[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY}, ss[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int64_t v = threadIdx.x; v < nvec; v += 256) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(row + v * 4);
      ms_add_f(mm[0], ss[0], x.x);
      ms_add_f(mm[1], ss[1], x.y);
      ms_add_f(mm[2], ss[2], x.z);
      ms_add_f(mm[3], ss[3], x.w);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) ms_merge_f(m, s, mm[j], ss[j]);
  }
  for (int64_t i = vend + threadIdx.x; i < vocab; i += 256) ms_add_f(m, s, row[i]);
  block_ms_f(m, s);
  const float lse = m + logf(s);
  const bool in_range = label >= 0 && label < vocab;
  const float target = (valid && in_range) ? row[label] : 0.0f;
  __syncthreads();  // the target is read before any write
  if (threadIdx.x == 0) row_loss[r] = !valid ? 0.0f : (in_range ? lse - target : __builtin_nanf(""));
  if constexpr (!kGrad) return;
  auto g_of = [&](float x, int64_t idx) -> float {
    if (!valid) return 0.0f;
    const float p = expf(x - lse);
    return idx == label ? p - 1.0f : p;
  };
  if (vec) {
    for (int64_t v = threadIdx.x; v < nvec; v += 256) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(row + v * 4);
      const int64_t b = v * 4;
      *reinterpret_cast<f32x4*>(row + b) = f32x4{g_of(x.x, b), g_of(x.y, b + 1), g_of(x.z, b + 2), g_of(x.w, b + 3)};
    }
  }
  for (int64_t i = vend + threadIdx.x; i < vocab; i += 256) row[i] = g_of(row[i], i);
}

// Fixed-order sums over rows: loss_sum, n_valid (count of label != ignore), mean.
__global__ __launch_bounds__(256) void ce_loss_kernel(const float* __restrict__ row_loss,
                                                      const int64_t* __restrict__ labels,
                                                      int64_t rows, int64_t ignore_index,
                                                      float* __restrict__ out3) {
  __shared__ double sl[4];
  __shared__ long long sn[4];
  double acc = 0.0;
  long long cnt = 0;
  for (int64_t i = threadIdx.x; i < rows; i += 256) {
    acc += static_cast<double>(row_loss[i]);
    cnt += labels[i] != ignore_index;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    acc += __shfl_xor(acc, off, 64);
    cnt += __shfl_xor(cnt, off, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    sl[threadIdx.x >> 6] = acc;
    sn[threadIdx.x >> 6] = cnt;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const double total = sl[0] + sl[1] + sl[2] + sl[3];
    long long n = sn[0] + sn[1] + sn[2] + sn[3];
    const float loss_sum = static_cast<float>(total);
    const float n_valid = static_cast<float>(n < 1 ? 1 : n);  // clamp_min(1)
    out3[0] = loss_sum;
    out3[1] = n_valid;
    out3[2] = loss_sum / n_valid;
  }
}

// Backward scaling, fused_linear_ce.py:117-126: grad_h (bf16) *= bf16(g / n_valid)
// (the scale is cast to the grad's dtype, then a bf16 multiply), grad_W *= g / n_valid.
__global__ __launch_bounds__(256) void ce_scale_kernel(uint16_t* __restrict__ gh, int64_t nh,
                                                       float* __restrict__ gw, int64_t nw,
                                                       const float* __restrict__ grad_out,
                                                       const float* __restrict__ n_valid) {
  const float scale = *grad_out / *n_valid;
  const float scale_b = __uint_as_float(rne16(scale) << 16);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < nh; i += stride)
    gh[i] = static_cast<uint16_t>(rne16(__uint_as_float(static_cast<uint32_t>(gh[i]) << 16) * scale_b));
  if (gw)
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < nw; i += stride)
      gw[i] = gw[i] * scale;
}

// grad_W hand-over (fused_linear_ce.py:80-81 for each chunk in order, and :126 with kScale):
// acc = ((((kAccumulate ? acc : +0) + float(c[0])) + float(c[1])) + ...) [* g / n_valid] over
// n chunks (1 to kMaxFold) in one pass. The reference adds each chunk into a zero-filled
// buffer (+0 + x also maps -0 to +0), so every element sees its fp32 operations in its order:
// the bits of one `+=` per chunk, then `mul_`, for one read and one write of the accumulator
// per n chunks. One wave per 256-element slice and one group of 4 per lane: each load or store
// instruction of the wave is one contiguous span (1 KiB of the fp32 accumulator, 512 B of each
// bf16 chunk), non-temporal, as in the optimizer's update. The slice that holds the end of a
// length not a multiple of 4, and every slice when a pointer is not aligned for the vectors,
// goes element by element.
constexpr int kMaxFold = 8;
struct FoldChunks {
  const uint16_t* p[kMaxFold];
};
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define CE_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ T ld_nt(const T* p) {
  return __builtin_nontemporal_load((const CE_GLOBAL T*)p);
}
template <typename T>
__device__ __forceinline__ void st_nt(T* p, T v) {
  __builtin_nontemporal_store(v, (CE_GLOBAL T*)p);
}

template <bool kAccumulate, bool kScale>
__global__ __launch_bounds__(64) void ce_grad_w_fold_kernel(float* __restrict__ acc, FoldChunks ch, int n,
                                                            int64_t nw, int64_t first_slice,
                                                            const float* __restrict__ grad_out,
                                                            const float* __restrict__ n_valid) {
  const float scale = kScale ? *grad_out / *n_valid : 1.0f;
  uint64_t misaligned = reinterpret_cast<uint64_t>(acc) & 15u;
#pragma unroll
  for (int c = 0; c < kMaxFold; ++c)
    if (c < n) misaligned |= reinterpret_cast<uint64_t>(ch.p[c]) & 7u;
  const int64_t e = (first_slice + blockIdx.x) * 256 + static_cast<int64_t>(threadIdx.x) * 4;
  if (misaligned == 0 && e + 4 <= nw) {
    u32x2 w[kMaxFold];
#pragma unroll
    for (int c = 0; c < kMaxFold; ++c)
      if (c < n) w[c] = ld_nt(reinterpret_cast<const u32x2*>(ch.p[c] + e));
    f32x4 a = kAccumulate ? ld_nt(reinterpret_cast<const f32x4*>(acc + e)) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < kMaxFold; ++c) {
      if (c < n) {
        a.x = a.x + lo16(w[c].x); a.y = a.y + hi16(w[c].x);
        a.z = a.z + lo16(w[c].y); a.w = a.w + hi16(w[c].y);
      }
    }
    if (kScale) {
      a.x = a.x * scale; a.y = a.y * scale; a.z = a.z * scale; a.w = a.w * scale;
    }
    st_nt(reinterpret_cast<f32x4*>(acc + e), a);
    return;
  }
  const int64_t end = e + 4 < nw ? e + 4 : nw;
  for (int64_t i = e; i < end; ++i) {
    float x = kAccumulate ? acc[i] : 0.0f;
#pragma unroll
    for (int c = 0; c < kMaxFold; ++c)
      if (c < n) x = x + __uint_as_float(static_cast<uint32_t>(ch.p[c][i]) << 16);
    if (kScale) x = x * scale;
    acc[i] = x;
  }
}

// Backward of fp32 hidden states, fused_linear_ce.py:68,80,120: the reference keeps grad_hidden
// in the hidden states' dtype, so under autocast its fp32 buffer holds the widened bf16 GEMM
// result (`grad_hidden[s:e] = gh`, -0 kept) and is scaled in fp32 (`mul_(scale)`):
// dst = float(src) * (g / n_valid).
__global__ __launch_bounds__(256) void ce_widen_scale_kernel(float* __restrict__ dst,
                                                             const uint16_t* __restrict__ src, int64_t n,
                                                             const float* __restrict__ grad_out,
                                                             const float* __restrict__ n_valid) {
  const float scale = *grad_out / *n_valid;
  const bool vec = ((reinterpret_cast<uint64_t>(dst) | reinterpret_cast<uint64_t>(src)) & 15u) == 0;
  const int64_t vend = vec ? (n & ~int64_t(7)) : 0;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256 * 8;
  for (int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 8; i < vend; i += stride) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(src + i);
    f32x4 a = {lo16(w.x), hi16(w.x), lo16(w.y), hi16(w.y)};
    f32x4 b = {lo16(w.z), hi16(w.z), lo16(w.w), hi16(w.w)};
    a.x = a.x * scale; a.y = a.y * scale; a.z = a.z * scale; a.w = a.w * scale;
    b.x = b.x * scale; b.y = b.y * scale; b.z = b.z * scale; b.w = b.w * scale;
    *reinterpret_cast<f32x4*>(dst + i) = a;
    *reinterpret_cast<f32x4*>(dst + i + 4) = b;
  }
  for (int64_t i = vend + static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256)
    dst[i] = __uint_as_float(static_cast<uint32_t>(src[i]) << 16) * scale;
}

int ce_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return ce_fail(TM_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return TM_OK;
}

// One block per row. The kernel (register or streaming path) depends only on the vocabulary,
// so the loss-only pass runs the same arithmetic as the gradient pass and gives the same bits.
template <bool kGrad>
int ce_rows_launch(uint16_t* d_logits, int64_t ld, const int64_t* d_labels, int64_t rows, int64_t vocab,
                   int64_t ignore_index, float* d_row_loss, void* stream, const char* who) {
  if (rows < 0 || vocab <= 0 || ld < vocab)
    return ce_fail(TM_EINVAL, "%s: bad sizes rows=%lld vocab=%lld ld=%lld", who, (long long)rows,
                   (long long)vocab, (long long)ld);
  if (rows == 0) return TM_OK;
  if (!d_logits || !d_labels || !d_row_loss) return ce_fail(TM_EINVAL, "%s: null pointer", who);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool regs = (vocab >> 3) <= static_cast<int64_t>(kRowThreadsRegs) * kRegCols;
  // a launch holds fewer than 2^32 work-items: longer row lists (small vocabularies in one
  // chunk) go in several launches
  const int64_t max_rows = 0xFFFFFFFFll / (regs ? kRowThreadsRegs : kRowThreadsStream);
  for (int64_t r0 = 0; r0 < rows; r0 += max_rows) {
    const uint32_t nr = static_cast<uint32_t>(rows - r0 < max_rows ? rows - r0 : max_rows);
    uint16_t* lg = d_logits + r0 * ld;
    if (regs)
      hipLaunchKernelGGL((ce_rows_kernel<true, kRowThreadsRegs, kGrad>), dim3(nr), dim3(kRowThreadsRegs), 0, s,
                         lg, ld, d_labels + r0, vocab, ignore_index, d_row_loss + r0);
    else
      hipLaunchKernelGGL((ce_rows_kernel<false, kRowThreadsStream, kGrad>), dim3(nr), dim3(kRowThreadsStream),
                         0, s, lg, ld, d_labels + r0, vocab, ignore_index, d_row_loss + r0);
    if (int rc = ce_check_launch(who)) return rc;
  }
  return TM_OK;
}

template <bool kGrad>
int ce_rows_f32_launch(float* d_logits, int64_t ld, const int64_t* d_labels, int64_t rows, int64_t vocab,
                       int64_t ignore_index, float* d_row_loss, void* stream, const char* who) {
  if (rows < 0 || vocab <= 0 || ld < vocab)
    return ce_fail(TM_EINVAL, "%s: bad sizes rows=%lld vocab=%lld ld=%lld", who, (long long)rows,
                   (long long)vocab, (long long)ld);
  if (rows == 0) return TM_OK;
  if (!d_logits || !d_labels || !d_row_loss) return ce_fail(TM_EINVAL, "%s: null pointer", who);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t max_rows = 0xFFFFFFFFll / 256;  // a launch holds fewer than 2^32 work-items
  for (int64_t r0 = 0; r0 < rows; r0 += max_rows) {
    const uint32_t nr = static_cast<uint32_t>(rows - r0 < max_rows ? rows - r0 : max_rows);
    hipLaunchKernelGGL((ce_rows_f32_kernel<kGrad>), dim3(nr), dim3(256), 0, s, d_logits + r0 * ld, ld,
                       d_labels + r0, vocab, ignore_index, d_row_loss + r0);
    if (int rc = ce_check_launch(who)) return rc;
  }
  return TM_OK;
}

// One ce_grad_w_fold_kernel pass over nw elements: one 64-thread workgroup per 256-element
// slice, over as many launches as the 2^32 work-item limit of a launch requires.
int fold_launch(float* d_grad_w, const FoldChunks& ch, int n_chunks, int64_t nw, int accumulate,
                const float* d_grad_out, const float* d_n_valid, void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool scale = d_grad_out != nullptr;
  const int64_t slices = (nw + 255) / 256;
  constexpr int64_t kMaxSlicesPerLaunch = int64_t(1) << 25;  // 2^31 work-items
  for (int64_t first = 0; first < slices; first += kMaxSlicesPerLaunch) {
    const int64_t count = slices - first < kMaxSlicesPerLaunch ? slices - first : kMaxSlicesPerLaunch;
    const dim3 grid(static_cast<uint32_t>(count)), block(64);
    if (accumulate && scale)
      hipLaunchKernelGGL((ce_grad_w_fold_kernel<true, true>), grid, block, 0, s, d_grad_w, ch, n_chunks, nw,
                         first, d_grad_out, d_n_valid);
    else if (accumulate)
      hipLaunchKernelGGL((ce_grad_w_fold_kernel<true, false>), grid, block, 0, s, d_grad_w, ch, n_chunks, nw,
                         first, d_grad_out, d_n_valid);
    else if (scale)
      hipLaunchKernelGGL((ce_grad_w_fold_kernel<false, true>), grid, block, 0, s, d_grad_w, ch, n_chunks, nw,
                         first, d_grad_out, d_n_valid);
    else
      hipLaunchKernelGGL((ce_grad_w_fold_kernel<false, false>), grid, block, 0, s, d_grad_w, ch, n_chunks, nw,
                         first, d_grad_out, d_n_valid);
    const int rc = ce_check_launch("ce_grad_w_fold_kernel");
    if (rc != TM_OK) return rc;
  }
  return TM_OK;
}

template <bool kTwo>
int ce_grad_w_launch(float* d_grad_w, const uint16_t* d_chunk, const uint16_t* d_chunk2, int64_t nw,
                     int accumulate, const float* d_grad_out, const float* d_n_valid, void* stream,
                     const char* who) {
  if (nw < 0) return ce_fail(TM_EINVAL, "%s: negative size", who);
  if (nw == 0) return TM_OK;
  if (!d_grad_w || !d_chunk || (kTwo && !d_chunk2) || (d_grad_out != nullptr) != (d_n_valid != nullptr))
    return ce_fail(TM_EINVAL, "%s: null pointer", who);
  FoldChunks ch = {};
  ch.p[0] = d_chunk;
  if (kTwo) ch.p[1] = d_chunk2;
  return fold_launch(d_grad_w, ch, kTwo ? 2 : 1, nw, accumulate, d_grad_out, d_n_valid, stream);
}

int ce_grad_w_fold_launch(float* d_grad_w, const uint16_t* const* h_chunks, int n_chunks, int64_t nw,
                          int accumulate, const float* d_grad_out, const float* d_n_valid, void* stream) {
  const char* who = "tm_ce_grad_w_fold";
  if (nw < 0 || n_chunks < 1 || n_chunks > kMaxFold)
    return ce_fail(TM_EINVAL, "%s: %d chunks (1 to %d) of %lld elements", who, n_chunks, kMaxFold, (long long)nw);
  if (!h_chunks || !d_grad_w || (d_grad_out != nullptr) != (d_n_valid != nullptr))
    return ce_fail(TM_EINVAL, "%s: null pointer", who);
  FoldChunks ch = {};
  for (int c = 0; c < n_chunks; ++c) {
    if (!h_chunks[c]) return ce_fail(TM_EINVAL, "%s: null chunk %d", who, c);
    ch.p[c] = h_chunks[c];
  }
  if (nw == 0) return TM_OK;
  return fold_launch(d_grad_w, ch, n_chunks, nw, accumulate, d_grad_out, d_n_valid, stream);
}

}  // namespace

extern "C" {

int tm_ce_rows_bf16(uint16_t* d_logits, int64_t ld, const int64_t* d_labels, int64_t rows,
                    int64_t vocab, int64_t ignore_index, float* d_row_loss, void* stream) {
  return ce_rows_launch<true>(d_logits, ld, d_labels, rows, vocab, ignore_index, d_row_loss, stream,
                              "tm_ce_rows_bf16");
}

int tm_ce_rows_loss_bf16(const uint16_t* d_logits, int64_t ld, const int64_t* d_labels, int64_t rows,
                         int64_t vocab, int64_t ignore_index, float* d_row_loss, void* stream) {
  // the kGrad=false kernels only read the logits
  return ce_rows_launch<false>(const_cast<uint16_t*>(d_logits), ld, d_labels, rows, vocab, ignore_index,
                               d_row_loss, stream, "tm_ce_rows_loss_bf16");
}

int tm_ce_rows_f32(float* d_logits, int64_t ld, const int64_t* d_labels, int64_t rows, int64_t vocab,
                   int64_t ignore_index, float* d_row_loss, void* stream) {
  return ce_rows_f32_launch<true>(d_logits, ld, d_labels, rows, vocab, ignore_index, d_row_loss, stream,
                                  "tm_ce_rows_f32");
}

int tm_ce_rows_loss_f32(const float* d_logits, int64_t ld, const int64_t* d_labels, int64_t rows, int64_t vocab,
                        int64_t ignore_index, float* d_row_loss, void* stream) {
  return ce_rows_f32_launch<false>(const_cast<float*>(d_logits), ld, d_labels, rows, vocab, ignore_index,
                                   d_row_loss, stream, "tm_ce_rows_loss_f32");
}

int tm_ce_loss(const float* d_row_loss, const int64_t* d_labels, int64_t rows, int64_t ignore_index,
               float* d_out3, void* stream) {
  if (rows < 0) return ce_fail(TM_EINVAL, "tm_ce_loss: negative rows");
  if (!d_out3 || (rows > 0 && (!d_row_loss || !d_labels)))
    return ce_fail(TM_EINVAL, "tm_ce_loss: null pointer");
  hipLaunchKernelGGL(ce_loss_kernel, dim3(1), dim3(256), 0, static_cast<hipStream_t>(stream),
                     d_row_loss, d_labels, rows, ignore_index, d_out3);
  return ce_check_launch("ce_loss_kernel");
}

int tm_ce_scale_grads(uint16_t* d_grad_h, int64_t nh, float* d_grad_w, int64_t nw,
                      const float* d_grad_out, const float* d_n_valid, void* stream) {
  if (nh < 0 || nw < 0) return ce_fail(TM_EINVAL, "tm_ce_scale_grads: negative size");
  if ((nh > 0 && !d_grad_h) || (nw > 0 && !d_grad_w) || !d_grad_out || !d_n_valid)
    return ce_fail(TM_EINVAL, "tm_ce_scale_grads: null pointer");
  int64_t n = nh > nw ? nh : nw;
  int64_t blocks = (n + 256 * 8 - 1) / (256 * 8);
  if (blocks < 1) blocks = 1;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(ce_scale_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), d_grad_h, nh, nw > 0 ? d_grad_w : nullptr, nw,
                     d_grad_out, d_n_valid);
  return ce_check_launch("ce_scale_kernel");
}

int tm_ce_grad_w(float* d_grad_w, const uint16_t* d_chunk, int64_t nw, int accumulate,
                 const float* d_grad_out, const float* d_n_valid, void* stream) {
  return ce_grad_w_launch<false>(d_grad_w, d_chunk, nullptr, nw, accumulate, d_grad_out, d_n_valid, stream,
                                 "tm_ce_grad_w");
}

int tm_ce_grad_w2(float* d_grad_w, const uint16_t* d_chunk, const uint16_t* d_chunk2, int64_t nw,
                  int accumulate, const float* d_grad_out, const float* d_n_valid, void* stream) {
  return ce_grad_w_launch<true>(d_grad_w, d_chunk, d_chunk2, nw, accumulate, d_grad_out, d_n_valid, stream,
                                "tm_ce_grad_w2");
}

int tm_ce_grad_w_fold(float* d_grad_w, const uint16_t* const* h_chunks, int n_chunks, int64_t nw, int accumulate,
                      const float* d_grad_out, const float* d_n_valid, void* stream) {
  return ce_grad_w_fold_launch(d_grad_w, h_chunks, n_chunks, nw, accumulate, d_grad_out, d_n_valid, stream);
}

int tm_ce_widen_scale(float* d_dst, const uint16_t* d_src, int64_t n, const float* d_grad_out,
                      const float* d_n_valid, void* stream) {
  if (n < 0) return ce_fail(TM_EINVAL, "tm_ce_widen_scale: negative size");
  if (n == 0) return TM_OK;
  if (!d_dst || !d_src || !d_grad_out || !d_n_valid) return ce_fail(TM_EINVAL, "tm_ce_widen_scale: null pointer");
  int64_t blocks = (n + 256 * 8 - 1) / (256 * 8);
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(ce_widen_scale_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), d_dst, d_src, n, d_grad_out, d_n_valid);
  return ce_check_launch("ce_widen_scale_kernel");
}

}  // extern "C"
