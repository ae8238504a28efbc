// tm_optim.hip -- gfx950 kernels and C ABI of the mixed-precision optimizer step.
//
// Kernels (all memory-bound, no MFMA):
//   norm_partials_kernel  pass 1 of the deterministic global grad norm: a fixed grid of
//                         TM_NORM_PARTIALS blocks, block b owns chunks b, b+G, ...; each
//                         writes one fp64 partial sum of squares (no atomics).
//   norm_finalize_kernel  pass 2: one block sums the partials in a fixed order, then
//                         sqrt and the clip coefficient, both on device.
//   adamw_prep_kernel     one thread per tensor: step += 1, bias corrections in fp64,
//                         per-tensor constants for the update.
//   adamw_update_kernel   one wave per 256-element slice of a chunk, on a grid shifted to
//                         the fp32 arrays' 1 KiB boundaries: reads grad, master, m, v once,
//                         writes master, m, v and the bf16 working copy once, 16-byte accesses.
//   grad_scale_kernel     eager in-place clip (grad *= coef), one wave per 512-element slice.
//   accumulate_list_kernel / accumulate_list_sumsq_kernel + slice_reduce_kernel
//                         fp32 accumulation buffers += bf16 micro-step grads over a list;
//                         on the last micro-step each slice also writes its fp64 sum of
//                         squares, which slice_reduce_kernel sums in the norm's fixed order.
//   accumulate_kernel     one fp32 accumulation buffer += bf16 micro-step grad.
//   cast_bf16_kernel      bf16 working copy = RNE(master).
//
// Arithmetic of the update follows torch's fused AdamW device functor
// (torch/include/ATen/native/hip/fused_adam_utils.cuh:22-92,106-199): hyper-parameters
// are double; the decay and both moment updates are evaluated in double and rounded
// to float; bias corrections are double, narrowed to float; the final division chain
// is float. Floating-point contraction is switched off for the whole file and every
// fused multiply-add is an explicit fma()/fmaf() call, so each rounding point is the
// one written here and the C oracle reproduces the result bit for bit. Division and
// sqrtf are the correctly rounded HIP defaults (never the native approximations).

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "torchure_amd.h"
#include "tm_internal.h"

#pragma clang fp contract(off)

namespace {
thread_local char g_err[512] = "";
}  // namespace

int tm_internal_fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

namespace {

constexpr int kThreads = 256;  // 4 wave64 per block
constexpr int kVec = 8;        // elements per thread per iteration (16 B of bf16)
constexpr int kWaves = kThreads / 64;
constexpr int kGroupSpan0 = kThreads * 4;  // elements covered by one 4-element group per thread

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <typename... A>
int fail(int code, const char* fmt, A... args) {
  return tm_internal_fail(code, fmt, args...);
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TM_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return TM_OK;
}

// Per-tensor constants produced by adamw_prep_kernel (64 bytes).
struct alignas(16) TensorScal {
  double neg_lrwd;  // -(lr * weight_decay)
  double beta1;
  double omb1;  // 1 - beta1
  double beta2;
  double omb2;  // 1 - beta2
  double eps;
  float step_size;  // float(lr / double(float(1 - beta1^step)))
  float bc2s;       // float(sqrt(1 - beta2^step))
  uint32_t decay;   // weight_decay != 0
  uint32_t mode;    // the update's per-tensor launch decisions (kMode* bits, grid phase)
};

// TensorScal::mode: bits 0-7 hold the grid phase (elements, a multiple of 4, below 256) of a
// tensor updated with 16-byte vectors; the rest are flags.
constexpr uint32_t kModePhase = 0xFFu;
constexpr uint32_t kModeVec = 1u << 8;    // every array aligned for the vector path
constexpr uint32_t kModeF32 = 1u << 9;    // fp32 grad (else bf16)
constexpr uint32_t kModeOut = 1u << 10;   // bf16 working copy written
constexpr uint32_t kModeClip = 1u << 11;  // TM_FLAG_CLIP set on the record

constexpr size_t kPartialBytes = sizeof(double) * TM_NORM_PARTIALS;

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// ---------------------------------------------------------------- element helpers

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ float bf16_at(const uint16_t* p, int64_t i) {
  return __uint_as_float(static_cast<uint32_t>(p[i]) << 16);
}

// Round-to-nearest-even fp32 -> bf16, NaN -> 0x7FC0
// (torch/include/torch/headeronly/util/BFloat16.h:100-114).
__device__ __forceinline__ uint32_t bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
  return (f != f) ? 0x7FC0u : r;
}

// Vector accesses go through global-address-space pointers. The arrays' addresses come
// from the tensor table as plain integers, so the compiler would otherwise emit FLAT
// instructions, which count in both vmcnt and lgkmcnt and can only be waited for all at
// once: every first use of a loaded value then drained every load and store in flight.
// Global instructions count in vmcnt only, in order, so a wave keeps its other loads and
// its stores outstanding while it computes (the update measured 0.3-0.5% faster in every
// HBM region; the mixed read/write stream, not the waits, bounds it). Every buffer here is
// device-visible global memory (never LDS or scratch), which global instructions address.
#define TM_GLOBAL __attribute__((address_space(1)))
template <bool kNT, typename T>
__device__ __forceinline__ T ld(const T* p) {
  const TM_GLOBAL T* g = (const TM_GLOBAL T*)p;
  if constexpr (kNT) return __builtin_nontemporal_load(g);
  else return *g;
}
template <bool kNT, typename T>
__device__ __forceinline__ void st(T* p, T v) {
  TM_GLOBAL T* g = (TM_GLOBAL T*)p;
  if constexpr (kNT) __builtin_nontemporal_store(v, g);
  else *g = v;
}

// One AdamW element. p, m, v are the fp32 values in memory; g is the (clipped) fp32
// grad. Statement by statement (fused_adam_utils.cuh line numbers):
//   :63-64  p = float(double(p) - (lr*wd) * double(p))           [if wd != 0]
//   :69     m = float(beta1 * double(m) + (1 - beta1) * double(g))
//   :70     v = float(beta2 * double(v) + (1 - beta2) * double(g) * double(g))
//   :77     denom = float(double(sqrtf(v) / bc2s) + eps)
//   :79     p = p - (step_size * m) / denom                       [float]
// The double sums are single fused multiply-adds (the contraction hipcc applies to
// the functor's expressions); the oracle uses the same fma() calls.
__device__ __forceinline__ void adamw_elem(float& p, float& m, float& v, float g,
                                           const TensorScal& c) {
  if (c.decay) {
    const double pd = static_cast<double>(p);
    p = static_cast<float>(fma(c.neg_lrwd, pd, pd));
  }
  const double gd = static_cast<double>(g);
  m = static_cast<float>(fma(c.beta1, static_cast<double>(m), c.omb1 * gd));
  v = static_cast<float>(fma(c.beta2, static_cast<double>(v), (c.omb2 * gd) * gd));
  const float q = sqrtf(v) / c.bc2s;
  const float denom = static_cast<float>(static_cast<double>(q) + c.eps);
  p = p - (c.step_size * m) / denom;
}

__device__ __forceinline__ bool aligned16(uint64_t a) { return (a & 15u) == 0; }
__device__ __forceinline__ bool aligned8(uint64_t a) { return (a & 7u) == 0; }

// ------------------------------------------------------------- one-wave slices
//
// The streaming kernels (update, eager scale, accumulation, cast) run one wave64 per
// workgroup, and each workgroup covers one slice of kSlice = 256 consecutive elements:
// 4 per lane, one 16-byte access per lane and fp32 array. A chunk of the chunk table is
// covered by chunk_elems / kSlice consecutive workgroups. Measured on MI355X over the same
// buffers, against one 256-thread workgroup looping over a whole 16,384-element chunk:
// the AdamW update moved its 28 B/param at 6.0 TB/s instead of 5.3, a 16-byte store stream
// ran at 6.6-7.2 TB/s instead of 5.2-5.7, and a copy at 6.5 TB/s instead of 5.1.
constexpr int kWave = 64;
constexpr int kSlice = kWave * 4;
// Dynamic LDS that the update launch requests and never uses. It caps a CU at 12
// resident update workgroups (12 x 13,312 B of gfx950's 160 KB; 13 would need 173,056 B, also
// with 512- or 1024-byte allocation granules), i.e. 3 waves per SIMD instead of as many as
// the wave slots hold (its 47 VGPRs do not limit them). Each update wave keeps eight 1 KB or
// 512 B streams in flight (28 B per element); with fewer such waves, fewer requests queue at
// the memory side. The 4B update then runs 6.39-6.46 TB/s on the process's first allocation
// and on a second one, against 5.65 and 6.07 TB/s uncapped (0.6B: 6.41-6.43 against
// 5.96-5.99). Caps of 11-14 workgroups per CU were within 3%; 10 and fewer were slower (8: 5.8
// TB/s, 5: 3.4). The lighter streams run uncapped. They move 4-10 B per element per wave (the
// eager scale, the cast, the accumulation), and the same cap halved their rates: the 4B cast
// 6.5 -> 3.3 TB/s, the accumulation 6.7 -> 4.3, the scale 4.7 -> 2.2.
constexpr int kUpdateLds = 13312;
// A launch holds fewer than 2^32 work-items: at most this many one-wave workgroups.
constexpr int64_t kMaxSliceBlocks = 0xFFFFFFFFll / kWave;

// Chunk and first element of this workgroup's slice, in a launch that starts at chunk
// first_chunk with slices_per_chunk = chunk_elems / kS workgroups per chunk. A power of two
// (64 at the default chunk size) takes a shift and a mask instead of the integer division,
// which costs about 25 instructions in every one-wave workgroup.
template <int kS = kSlice>
__device__ __forceinline__ void slice_of(const tm_chunk_t* __restrict__ chunks, uint32_t first_chunk,
                                         uint32_t slices_per_chunk, int64_t chunk_elems,
                                         tm_chunk_t& ck, int64_t& start) {
  uint32_t local, sub;
  if ((slices_per_chunk & (slices_per_chunk - 1)) == 0) {
    local = blockIdx.x >> __builtin_ctz(slices_per_chunk);
    sub = blockIdx.x & (slices_per_chunk - 1);
  } else {
    local = blockIdx.x / slices_per_chunk;
    sub = blockIdx.x - local * slices_per_chunk;
  }
  ck = chunks[first_chunk + local];
  start = static_cast<int64_t>(ck.chunk) * chunk_elems + static_cast<int64_t>(sub) * kS;
}

// Policy::group(e) / Policy::one(i) over the slice [start, end): lane t takes the group
// [start + 4t, +4) when vec is set, and the rest of the slice goes element by element.
template <class Policy>
__device__ __forceinline__ void slice_apply(const Policy& pol, int64_t start, int64_t end, bool vec) {
  int64_t vend = start;
  if (vec) {
    vend = start + ((end - start) & ~int64_t(3));
    const int64_t e = start + static_cast<int64_t>(threadIdx.x) * 4;
    if (e < vend) pol.group(e);
  }
  for (int64_t i = vend + threadIdx.x; i < end; i += kWave) pol.one(i);
}

// ------------------------------------------------------------------- reductions

__device__ __forceinline__ double wave_sum(double x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// Fixed-order block sum; the result is valid in thread 0.
__device__ __forceinline__ double block_sum(double x) {
  __shared__ double lds[kWaves];
  x = wave_sum(x);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  if (lane == 0) lds[wave] = x;
  __syncthreads();
  double s = 0.0;
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 0; w < kWaves; ++w) s += lds[w];
  }
  return s;
}

// ------------------------------------------------------- fp32 sum of squares: slice order
//
// Every fp32 sum of squares (the norm of fp32 grads, and the norm fused into the last
// micro-step of grad accumulation) is formed in this one fixed order, so the fused and the
// standalone norm give identical bits:
//   slice partial: a chunk is cut into slices of kSlice = 256 elements. Over a slice
//     [start, end), lane t of a wave takes the group [start + 4t, +4) when the fp32 buffer is
//     16-byte aligned (sumsq4: its 4 squares fma-chained in fp64 from 0.0), then the elements
//     vend + t, vend + t + 64, ... of the slice's tail (all of the slice when the buffer is not
//     aligned), each fma'd onto the same lane sum; wave_sum then reduces the 64 lane sums in
//     its fixed tree (slice_wave_sum);
//   chunk total: lane t adds the chunk's slice partials t, t + 64, t + 128, ... in order,
//     starting from 0.0 (slices past the tensor's end count as 0.0), then slice_wave_sum;
//   block total: block b of the fixed grid of TM_NORM_PARTIALS adds the totals of its chunks
//     b, b + G, ... in order, starting from 0.0.
// norm_partials_kernel computes the slice partials itself (4 waves per block, through LDS);
// the fused accumulation runs one wave per slice, writes each slice partial to a workspace
// and slice_reduce_kernel forms the chunk and block totals from them.
// Policy::group(e) produces the 4 fp32 values at e (and may store them);
// Policy::one(i) produces one value.

constexpr int kSliceGroup = 64;  // slice partials a chunk total adds per lane round

// The fixed reduction tree of the slice order over the 64 lanes of a wave, on DPP moves
// within rows of 16 lanes and four lane reads (an xor-shuffle tree of doubles went through
// LDS permutes, and formed once per KiB of fp32 grads it slowed the standalone norm by a
// fifth): lanes i and i^1, then i and i^2 (each quad's sum in its 4 lanes), then the
// half-row mirror (two quads), the row mirror (the row's 16 lanes; each pair adds the same two
// values, so every lane of a row holds the same bits), then ((row0 + row1) + row2) + row3.
// Every lane of the wave must be active; every lane returns the same value.
template <int kCtrl>
__device__ __forceinline__ double dpp_f64(double x) {
  const uint64_t u = static_cast<uint64_t>(__double_as_longlong(x));
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(u)), kCtrl, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(u >> 32)), kCtrl, 0xF, 0xF,
                                             false);
  return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                                                     static_cast<uint32_t>(lo)));
}

__device__ __forceinline__ double lane_f64(double x, int lane) {
  const uint64_t u = static_cast<uint64_t>(__double_as_longlong(x));
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(u)), lane));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(u >> 32)), lane));
  return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
}

__device__ __forceinline__ double slice_wave_sum(double x) {
  x = x + dpp_f64<0xB1>(x);   // quad_perm [1,0,3,2]: lane i^1
  x = x + dpp_f64<0x4E>(x);   // quad_perm [2,3,0,1]: lane i^2
  x = x + dpp_f64<0x141>(x);  // row_half_mirror: lane 7 - i within 8
  x = x + dpp_f64<0x140>(x);  // row_mirror: lane 15 - i within 16
  return ((lane_f64(x, 0) + lane_f64(x, 16)) + lane_f64(x, 32)) + lane_f64(x, 48);
}

__device__ __forceinline__ double sumsq4(const f32x4 a, double s) {
  s = fma((double)a.x, (double)a.x, s);
  s = fma((double)a.y, (double)a.y, s);
  s = fma((double)a.z, (double)a.z, s);
  s = fma((double)a.w, (double)a.w, s);
  return s;
}

// The slice partial of [start, end) (end - start <= kSlice), the same value in every lane.
template <class Policy>
__device__ __forceinline__ double slice_sumsq(const Policy& pol, int64_t start, int64_t end, bool vec) {
  const int lane = threadIdx.x & 63;
  double s = 0.0;
  int64_t vend = start;
  if (vec) {
    vend = start + ((end - start) & ~int64_t(3));
    const int64_t e = start + static_cast<int64_t>(lane) * 4;
    if (e < vend) s = sumsq4(pol.group(e), s);
  }
  for (int64_t i = vend + lane; i < end; i += kWave) {
    const double x = pol.one(i);
    s = fma(x, x, s);
  }
  return slice_wave_sum(s);
}

struct ReadF32 {
  const float* g;
  __device__ __forceinline__ f32x4 group(int64_t e) const {
    return ld<true>(reinterpret_cast<const f32x4*>(g + e));
  }
  __device__ __forceinline__ float one(int64_t i) const { return g[i]; }
};

// The 4 bf16 values at micro + e widened: one 8-byte load when micro is 8-byte aligned,
// else four 2-byte loads (the lane still owns the same 4 elements).
__device__ __forceinline__ f32x4 micro4(const uint16_t* micro, int64_t e, bool mvec) {
  if (mvec) {
    const u32x2 w = ld<true>(reinterpret_cast<const u32x2*>(micro + e));
    return f32x4{bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y)};
  }
  return f32x4{bf16_at(micro, e), bf16_at(micro, e + 1), bf16_at(micro, e + 2), bf16_at(micro, e + 3)};
}

// acc (fp32) += micro (bf16), stored back; yields the new accumulator values.
struct AccumBf16 {
  float* acc;
  const uint16_t* micro;
  bool mvec;
  __device__ __forceinline__ f32x4 group(int64_t e) const {
    f32x4 a = ld<true>(reinterpret_cast<const f32x4*>(acc + e));
    const f32x4 m = micro4(micro, e, mvec);
    a.x = a.x + m.x;
    a.y = a.y + m.y;
    a.z = a.z + m.z;
    a.w = a.w + m.w;
    st<true>(reinterpret_cast<f32x4*>(acc + e), a);
    return a;
  }
  __device__ __forceinline__ float one(int64_t i) const {
    const float a = acc[i] + bf16_at(micro, i);
    acc[i] = a;
    return a;
  }
};

// acc (fp32) = micro (bf16) widened, stored without reading acc: the first micro-step,
// where autograd assigns the grad rather than adding it (so -0 stays -0).
struct AssignBf16 {
  float* acc;
  const uint16_t* micro;
  bool mvec;
  __device__ __forceinline__ f32x4 group(int64_t e) const {
    const f32x4 a = micro4(micro, e, mvec);
    st<true>(reinterpret_cast<f32x4*>(acc + e), a);
    return a;
  }
  __device__ __forceinline__ float one(int64_t i) const {
    const float a = bf16_at(micro, i);
    acc[i] = a;
    return a;
  }
};

// ------------------------------------------------------------------- norm pass 1

// The chunk total of an fp32 buffer in the slice order, formed by a kThreads-thread block:
// in each round of kSliceGroup slices, wave w forms the slice partials w, w + 4, ..., four at
// a time with their loads issued together, and parks them in sp (LDS); wave 0's lane t then
// adds partial t of the round. Valid in every lane of wave 0. Called by whole blocks only.
__device__ __forceinline__ double chunk_total_f32(const float* g, int64_t start, int64_t end, int64_t spc,
                                                  bool vec, double* sp) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const ReadF32 pol{g};
  double lane_acc = 0.0;
  for (int64_t g0 = 0; g0 < spc; g0 += kSliceGroup) {
#pragma unroll 1
    for (int b = 0; b < kSliceGroup / (4 * kWaves); ++b) {
      const int k0 = wave + kWaves * 4 * b;  // this batch's slices: k0, k0 + kWaves, ...
      f32x4 v[4];
      unsigned full = 0;  // whole aligned slices, read together
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t j = g0 + k0 + kWaves * u;
        const int64_t s0 = start + j * kSlice;
        if (vec && j < spc && s0 + kSlice <= end) {
          full |= 1u << u;
          v[u] = pol.group(s0 + static_cast<int64_t>(lane) * 4);
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (full & (1u << u)) {
          const double p = slice_wave_sum(sumsq4(v[u], 0.0));
          if (lane == 0) sp[k0 + kWaves * u] = p;
        }
      }
#pragma unroll 1
      for (int u = 0; u < 4; ++u) {  // a tensor's last slice, unaligned buffers, past the end
        if (full & (1u << u)) continue;
        const int64_t j = g0 + k0 + kWaves * u;
        const int64_t s0 = start + j * kSlice;
        const double p = (j < spc && s0 < end) ? slice_sumsq(pol, s0, min(s0 + kSlice, end), vec) : 0.0;
        if (lane == 0) sp[k0 + kWaves * u] = p;
      }
    }
    __syncthreads();
    if (wave == 0) lane_acc += sp[lane];
    __syncthreads();
  }
  return slice_wave_sum(lane_acc);
}

__global__ __launch_bounds__(kThreads) void norm_partials_kernel(
    const tm_tensor_t* __restrict__ tensors, int64_t n_tensors,
    const tm_chunk_t* __restrict__ chunks, int64_t n_chunks, int64_t chunk_elems,
    double* __restrict__ partials) {
  __shared__ double sp[kSliceGroup];
  double acc = 0.0;        // bf16 grads: this thread's share
  double f32_total = 0.0;  // fp32 grads: the block total of their chunk totals (wave 0)
  const int64_t spc = chunk_elems / kSlice;
  for (int64_t c = blockIdx.x; c < n_chunks; c += gridDim.x) {
    const tm_chunk_t ck = chunks[c];
    if (ck.tensor >= n_tensors) continue;
    const tm_tensor_t d = tensors[ck.tensor];
    const int64_t start = static_cast<int64_t>(ck.chunk) * chunk_elems;
    if (start >= d.numel) continue;
    const int64_t end = min(start + chunk_elems, d.numel);
    if (d.flags & TM_GRAD_F32) {  // block-uniform: the whole block takes this chunk
      const double t = chunk_total_f32(reinterpret_cast<const float*>(d.grad), start, end, spc,
                                       aligned16(d.grad), sp);
      if (threadIdx.x < kWave) f32_total += t;
    } else {
      const uint16_t* __restrict__ g = reinterpret_cast<const uint16_t*>(d.grad);
      if (aligned16(d.grad)) {
        const int64_t vend = start + ((end - start) & ~int64_t(kVec - 1));
        for (int64_t i = start + threadIdx.x * kVec; i < vend; i += kThreads * kVec) {
          const u32x4 w = ld<true>(reinterpret_cast<const u32x4*>(g + i));
          // bf16 squares are exact in fp32 (8-bit significands); 8 of them are summed
          // in fp32 and the group sum is accumulated in fp64.
          float s = 0.f;
          float x;
          x = bf16_lo(w.x); s = fmaf(x, x, s);
          x = bf16_hi(w.x); s = fmaf(x, x, s);
          x = bf16_lo(w.y); s = fmaf(x, x, s);
          x = bf16_hi(w.y); s = fmaf(x, x, s);
          x = bf16_lo(w.z); s = fmaf(x, x, s);
          x = bf16_hi(w.z); s = fmaf(x, x, s);
          x = bf16_lo(w.w); s = fmaf(x, x, s);
          x = bf16_hi(w.w); s = fmaf(x, x, s);
          acc += static_cast<double>(s);
        }
        for (int64_t i = vend + threadIdx.x; i < end; i += kThreads) {
          const double x = bf16_at(g, i);
          acc = fma(x, x, acc);
        }
      } else {
        for (int64_t i = start + threadIdx.x; i < end; i += kThreads) {
          const double x = bf16_at(g, i);
          acc = fma(x, x, acc);
        }
      }
    }
  }
  const double s = block_sum(acc);
  if (threadIdx.x == 0) partials[blockIdx.x] = s + f32_total;
}

// ------------------------------------------------------------------- norm pass 2

// clip coefficient of torchure/core/grad_helper.py:32, evaluated as torch evaluates
// `max_norm / (total + 1e-6)` on a 0-d fp32 tensor: fp32 add of 1e-6f, fp32
// reciprocal, fp32 multiply by float(max_norm), then clamp(max=1) with NaN passing
// through (torch/_tensor.py:1119-1122).
__device__ __forceinline__ float clip_coef(float norm, float max_norm) {
  const float r = 1.0f / (norm + 1e-6f);
  const float c = r * max_norm;
  return (c > 1.0f) ? 1.0f : c;
}

__global__ __launch_bounds__(kThreads) void norm_finalize_kernel(
    const double* __restrict__ partials, float max_norm, int clip, float* __restrict__ norm_out,
    float* __restrict__ coef_out) {
  double acc = 0.0;
  for (int i = threadIdx.x; i < TM_NORM_PARTIALS; i += kThreads) acc += partials[i];
  const double total = block_sum(acc);
  if (threadIdx.x == 0) {
    // The reference's norms reduce in fp32 (torch._foreach_norm, then vector_norm of the
    // stack): once the sum of squares rounds past FLT_MAX they return inf, and the clip
    // coefficient becomes 0. The fp64 sum here would stay finite, so it is cut at the same
    // point: 2^128 - 2^103, the smallest value fp32 rounding sends to infinity.
    const float norm = total >= 0x1.ffffffp+127 ? INFINITY : static_cast<float>(sqrt(total));
    *norm_out = norm;
    if (clip) *coef_out = clip_coef(norm, max_norm);
  }
}

__global__ void clip_coef_kernel(const float* __restrict__ norm, float max_norm,
                                 float* __restrict__ coef_out) {
  if (threadIdx.x == 0 && blockIdx.x == 0) *coef_out = clip_coef(*norm, max_norm);
}

// ------------------------------------------------------------------- grad scale

// The eager scale covers 512 elements per wave: lane t takes the groups [start + 4t, +4) and
// [start + 256 + 4t, +4), whose loads are both issued before either store. Each wave
// instruction is still one contiguous span (1 KiB of fp32, 512 B of bf16). With 256 elements
// per wave a bf16 scale moved 1 KiB per workgroup and ran at 4.8 TB/s on MI355X; with 512,
// 6.75 TB/s (2^31 bf16 elements, read and written in place).
constexpr int kScaleSlice = 2 * kSlice;
static_assert(TM_CHUNK_ALIGN % kScaleSlice == 0, "a chunk must hold whole scale slices");

struct ScaleF32 {
  float* g;
  float coef;
  typedef f32x4 Raw;
  __device__ __forceinline__ Raw load(int64_t e) const { return ld<true>(reinterpret_cast<const f32x4*>(g + e)); }
  __device__ __forceinline__ void finish(Raw a, int64_t e) const {
    a.x = a.x * coef;
    a.y = a.y * coef;
    a.z = a.z * coef;
    a.w = a.w * coef;
    st<true>(reinterpret_cast<f32x4*>(g + e), a);
  }
  __device__ __forceinline__ void one(int64_t i) const { g[i] = g[i] * coef; }
};

// torch._foreach_mul_ on a bf16 list holds the 0-d scalar in the list's dtype
// (BinaryOpScalarTensorFunctor, torch/include/ATen/native/hip/ForeachFunctors.cuh:309-342):
// the coefficient is rounded to bf16 (coef_b) before the fp32 multiply.
struct ScaleBf16 {
  uint16_t* g;
  float coef_b;
  typedef u32x2 Raw;
  __device__ __forceinline__ uint32_t scale2(uint32_t w) const {
    return bf16_rne(bf16_lo(w) * coef_b) | (bf16_rne(bf16_hi(w) * coef_b) << 16);
  }
  __device__ __forceinline__ Raw load(int64_t e) const { return ld<true>(reinterpret_cast<const u32x2*>(g + e)); }
  __device__ __forceinline__ void finish(Raw w, int64_t e) const {
    w.x = scale2(w.x);
    w.y = scale2(w.y);
    st<true>(reinterpret_cast<u32x2*>(g + e), w);
  }
  __device__ __forceinline__ void one(int64_t i) const {
    g[i] = static_cast<uint16_t>(bf16_rne(bf16_at(g, i) * coef_b));
  }
};

// Policy::load / finish over the two groups of a kScaleSlice slice [start, end) when vec is
// set; the rest of the slice goes element by element.
template <class Policy>
__device__ __forceinline__ void slice_apply2(const Policy& pol, int64_t start, int64_t end, bool vec) {
  int64_t vend = start;
  if (vec) {
    vend = start + ((end - start) & ~int64_t(3));
    const int64_t e0 = start + static_cast<int64_t>(threadIdx.x) * 4;
    const int64_t e1 = e0 + kSlice;
    const bool has0 = e0 < vend, has1 = e1 < vend;
    typename Policy::Raw r0{}, r1{};
    if (has0) r0 = pol.load(e0);
    if (has1) r1 = pol.load(e1);
    if (has0) pol.finish(r0, e0);
    if (has1) pol.finish(r1, e1);
  }
  for (int64_t i = vend + threadIdx.x; i < end; i += kWave) pol.one(i);
}

// One kScaleSlice slice per wave; the same single multiply per element on the vector and the
// element-wise path (16-byte fp32 / 8-byte bf16 vectors where the grad is so aligned).
__global__ __launch_bounds__(kWave) void grad_scale_kernel(
    const tm_tensor_t* __restrict__ tensors, int64_t n_tensors,
    const tm_chunk_t* __restrict__ chunks, uint32_t first_chunk, uint32_t slices_per_chunk,
    int64_t chunk_elems, const float* __restrict__ coef_p) {
  tm_chunk_t ck;
  int64_t start;
  slice_of<kScaleSlice>(chunks, first_chunk, slices_per_chunk, chunk_elems, ck, start);
  if (ck.tensor >= n_tensors) return;
  const tm_tensor_t d = tensors[ck.tensor];
  if (start >= d.numel) return;
  const int64_t end = min(start + kScaleSlice, d.numel);
  const float coef = *coef_p;
  if (d.flags & TM_GRAD_F32) {
    slice_apply2(ScaleF32{reinterpret_cast<float*>(d.grad), coef}, start, end, aligned16(d.grad));
  } else {
    const float coef_b = __uint_as_float(bf16_rne(coef) << 16);
    slice_apply2(ScaleBf16{reinterpret_cast<uint16_t*>(d.grad), coef_b}, start, end, aligned8(d.grad));
  }
}

// ------------------------------------------------------------------- AdamW prep

struct HyperArgs {
  tm_hyper_t g[TM_MAX_GROUPS];
  int32_t n;
};

// step += 1 and the per-tensor constants (fused_adam_utils.cuh:128-139; adam.py:877).
// Elements from the 1 KiB boundary at or before a 16-byte aligned fp32 array's start to that
// start (a multiple of 4, below kSlice): element e sits e + phase elements past the boundary.
__device__ __forceinline__ uint32_t fp32_phase(uint64_t a) {
  return static_cast<uint32_t>((a >> 2) & static_cast<uint64_t>(kSlice - 1));
}

// The update's decisions for one tensor, made once here instead of in each of its slices'
// workgroups: whether all its arrays take 16-byte vectors, its grad type, whether a bf16 copy
// is written, its clip flag, and its grid phase (adamw_update_kernel): the phase of the
// master, or that of m and v where those two agree and outvote it.
__device__ __forceinline__ uint32_t update_mode(const tm_tensor_t& d) {
  const bool f32 = (d.flags & TM_GRAD_F32) != 0;
  const bool out = d.param_bf16 != 0;
  uint32_t mode = (f32 ? kModeF32 : 0u) | (out ? kModeOut : 0u) | ((d.flags & TM_FLAG_CLIP) ? kModeClip : 0u);
  const bool grad_ok = f32 ? aligned16(d.grad) : aligned8(d.grad);
  if (aligned16(d.master) && aligned16(d.exp_avg) && aligned16(d.exp_avg_sq) && grad_ok &&
      (!out || aligned8(d.param_bf16))) {
    const uint32_t pp = fp32_phase(d.master), pm = fp32_phase(d.exp_avg), pv = fp32_phase(d.exp_avg_sq);
    const bool mv = pm == pv && pp != pm && !(f32 && fp32_phase(d.grad) == pp);
    mode |= kModeVec | (mv ? pm : pp);
  }
  return mode;
}

__global__ __launch_bounds__(kThreads) void adamw_prep_kernel(
    const tm_tensor_t* __restrict__ tensors, int64_t n_tensors, HyperArgs hyper,
    TensorScal* __restrict__ scal) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (t >= n_tensors) return;
  const tm_tensor_t d = tensors[t];
  const int32_t gi = d.group;
  float* step_p = reinterpret_cast<float*>(d.step);
  if (gi < 0 || gi >= hyper.n) {
    // A record naming a group the call does not have: the records live in device memory, so
    // the host cannot refuse it without a synchronisation. The tensor is poisoned instead of
    // stepped with another group's hyper-parameters: its step counter becomes NaN, and NaN
    // constants make the update write NaN into its master, moments and bf16 copy.
    const double nan = __builtin_nan("");
    *step_p = __builtin_nanf("");
    scal[t] = TensorScal{nan, nan, nan, nan, nan, nan, __builtin_nanf(""), __builtin_nanf(""), 1u,
                         (d.param_bf16 != 0 ? kModeOut : 0u) | ((d.flags & TM_GRAD_F32) ? kModeF32 : 0u)};
    return;
  }
  const tm_hyper_t h = hyper.g[gi];
  const float step = *step_p + 1.0f;
  *step_p = step;
  const double bc1 = 1.0 - pow(h.beta1, static_cast<double>(step));
  const double bc2 = 1.0 - pow(h.beta2, static_cast<double>(step));
  const float bc1f = static_cast<float>(bc1);
  TensorScal s;
  s.neg_lrwd = -(h.lr * h.weight_decay);
  s.beta1 = h.beta1;
  s.omb1 = 1.0 - h.beta1;
  s.beta2 = h.beta2;
  s.omb2 = 1.0 - h.beta2;
  s.eps = h.eps;
  s.step_size = static_cast<float>(h.lr / static_cast<double>(bc1f));
  s.bc2s = static_cast<float>(sqrt(bc2));
  s.decay = h.weight_decay != 0.0;
  s.mode = update_mode(d);
  scal[t] = s;
}

// ------------------------------------------------------------------- AdamW update

// Lane mapping. A lane owns one group of 4 consecutive elements: lane t of the wave that
// covers a slice starting at virtual position `start` takes [start + 4t - ph, +4), ph being
// the tensor's grid phase (below). Each load or store instruction of the wave is one
// contiguous span (1 KiB of an fp32 array, 512 B of a bf16 array) of whole cache lines when
// the arrays sit on those boundaries, so the stores leave no partially written lines behind. All accesses are
// non-temporal: the streams are touched once (measured 7% faster than temporal accesses).
struct Group4 {
  f32x4 p, m, v;
  float g[4];
};

template <bool kGradF32>
__device__ __forceinline__ void load_group(Group4& r, const tm_tensor_t& d, int64_t e) {
  if constexpr (kGradF32) {
    const f32x4 a = ld<true>(reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(d.grad) + e));
    r.g[0] = a.x; r.g[1] = a.y; r.g[2] = a.z; r.g[3] = a.w;
  } else {
    const u32x2 w =
        ld<true>(reinterpret_cast<const u32x2*>(reinterpret_cast<const uint16_t*>(d.grad) + e));
    r.g[0] = bf16_lo(w.x); r.g[1] = bf16_hi(w.x); r.g[2] = bf16_lo(w.y); r.g[3] = bf16_hi(w.y);
  }
  r.p = ld<true>(reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(d.master) + e));
  r.m = ld<true>(reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(d.exp_avg) + e));
  r.v = ld<true>(reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(d.exp_avg_sq) + e));
}

__device__ __forceinline__ void compute_group(Group4& r, const TensorScal& c, bool clip, float coef) {
  float p[4] = {r.p.x, r.p.y, r.p.z, r.p.w};
  float m[4] = {r.m.x, r.m.y, r.m.z, r.m.w};
  float v[4] = {r.v.x, r.v.y, r.v.z, r.v.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float gj = clip ? r.g[j] * coef : r.g[j];
    adamw_elem(p[j], m[j], v[j], gj, c);
  }
  r.p = f32x4{p[0], p[1], p[2], p[3]};
  r.m = f32x4{m[0], m[1], m[2], m[3]};
  r.v = f32x4{v[0], v[1], v[2], v[3]};
}

template <bool kOut>
__device__ __forceinline__ void store_group(const Group4& r, const tm_tensor_t& d, int64_t e) {
  st<true>(reinterpret_cast<f32x4*>(reinterpret_cast<float*>(d.master) + e), r.p);
  st<true>(reinterpret_cast<f32x4*>(reinterpret_cast<float*>(d.exp_avg) + e), r.m);
  st<true>(reinterpret_cast<f32x4*>(reinterpret_cast<float*>(d.exp_avg_sq) + e), r.v);
  if constexpr (kOut) {
    u32x2 o;
    o.x = bf16_rne(r.p.x) | (bf16_rne(r.p.y) << 16);
    o.y = bf16_rne(r.p.z) | (bf16_rne(r.p.w) << 16);
    st<true>(reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(d.param_bf16) + e), o);
  }
}

template <bool kGradF32, bool kOut>
__device__ __forceinline__ void update_group(const tm_tensor_t& d, int64_t e, const TensorScal& c,
                                             bool clip, float coef) {
  Group4 r;
  load_group<kGradF32>(r, d, e);
  compute_group(r, c, clip, coef);
  store_group<kOut>(r, d, e);
}

// Element-at-a-time path for whole tensors whose fp32 pointers are not 16-byte aligned
// (or bf16 pointers not 8-byte aligned). Lane t takes elements start + t, start + t + 64, ...
__device__ __forceinline__ void update_scalar(const tm_tensor_t& d, int64_t start, int64_t end,
                                              const TensorScal& c, bool clip, float coef) {
  float* P = reinterpret_cast<float*>(d.master);
  float* M = reinterpret_cast<float*>(d.exp_avg);
  float* V = reinterpret_cast<float*>(d.exp_avg_sq);
  uint16_t* O = reinterpret_cast<uint16_t*>(d.param_bf16);
  const bool f32 = (d.flags & TM_GRAD_F32) != 0;
  for (int64_t i = start + threadIdx.x; i < end; i += kWave) {
    float g = f32 ? reinterpret_cast<const float*>(d.grad)[i]
                  : bf16_at(reinterpret_cast<const uint16_t*>(d.grad), i);
    if (clip) g = g * coef;
    float p = P[i], m = M[i], v = V[i];
    adamw_elem(p, m, v, g, c);
    P[i] = p;
    M[i] = m;
    V[i] = v;
    if (O) O[i] = static_cast<uint16_t>(bf16_rne(p));
  }
}

// The elements [e, n) of one lane's last, partial group of 4 (a tensor whose length is not
// a multiple of 4), element by element by that lane alone.
__device__ __forceinline__ void update_lane_tail(const tm_tensor_t& d, int64_t e, int64_t n,
                                                 const TensorScal& c, bool clip, float coef) {
  float* P = reinterpret_cast<float*>(d.master);
  float* M = reinterpret_cast<float*>(d.exp_avg);
  float* V = reinterpret_cast<float*>(d.exp_avg_sq);
  uint16_t* O = reinterpret_cast<uint16_t*>(d.param_bf16);
  const bool f32 = (d.flags & TM_GRAD_F32) != 0;
  for (int64_t i = e; i < n; ++i) {
    float g = f32 ? reinterpret_cast<const float*>(d.grad)[i]
                  : bf16_at(reinterpret_cast<const uint16_t*>(d.grad), i);
    if (clip) g = g * coef;
    float p = P[i], m = M[i], v = V[i];
    adamw_elem(p, m, v, g, c);
    P[i] = p;
    M[i] = m;
    V[i] = v;
    if (O) O[i] = static_cast<uint16_t>(bf16_rne(p));
  }
}

// Slice grid on 1 KiB boundaries. A wave's fp32 access is one 1 KiB span per array; measured on
// MI355X (4e9 elements, the same memory viewed at other offsets), the update runs about 1.5%
// slower for each of master, m and v whose spans are not 1 KiB aligned (5.7% for all three),
// while the bf16 arrays' 512-byte spans cost nothing off their boundary. So a tensor is covered
// in a shifted grid: element e sits at virtual position e + ph, where ph is the phase (above)
// of the master, or that of m and v where those two agree and outvote it, so that virtual
// slice s, the elements [256 s - ph, 256 s + 256 - ph), starts on a 1 KiB boundary of the
// arrays that have that phase. The chunk table still gives the tensor
// ceil(n / chunk_elems) chunks, which cover virtual [0, covered) with covered = that count
// times chunk_elems; the last L = n + ph - covered elements (L <= ph) fall past it and take the
// first L virtual positions of slice 0, which the shift left empty. Every element lands in
// exactly one lane's group of 4, whose fp32 addresses stay 16-byte aligned.
__global__ __launch_bounds__(kWave) void adamw_update_kernel(
    const tm_tensor_t* __restrict__ tensors, int64_t n_tensors,
    const tm_chunk_t* __restrict__ chunks, uint32_t first_chunk, uint32_t slices_per_chunk,
    int64_t chunk_elems, const TensorScal* __restrict__ scal, const float* __restrict__ coef_p) {
  tm_chunk_t ck;
  int64_t start;
  slice_of(chunks, first_chunk, slices_per_chunk, chunk_elems, ck, start);
  if (ck.tensor >= n_tensors) return;
  const tm_tensor_t d = tensors[ck.tensor];
  const TensorScal c = scal[ck.tensor];
  const int64_t n = d.numel;
  const uint32_t mode = c.mode;
  const bool clip = (mode & kModeClip) && coef_p != nullptr;
  if (!(mode & kModeVec)) {  // element at a time, unshifted
    if (start >= n) return;
    update_scalar(d, start, min(start + kSlice, n), c, clip, clip ? *coef_p : 1.0f);
    return;
  }
  const int64_t ph = mode & kModePhase;
  if (start - ph >= n && start > 0) return;
  const float coef = clip ? *coef_p : 1.0f;
  int64_t e = start + static_cast<int64_t>(threadIdx.x) * 4 - ph;
  if (e < 0) e += (n + chunk_elems - 1) / chunk_elems * chunk_elems;  // slice 0's wrapped tail
  if (e + 4 <= n) {
    if (mode & kModeF32) {
      if (mode & kModeOut) update_group<true, true>(d, e, c, clip, coef);
      else update_group<true, false>(d, e, c, clip, coef);
    } else {
      if (mode & kModeOut) update_group<false, true>(d, e, c, clip, coef);
      else update_group<false, false>(d, e, c, clip, coef);
    }
  } else if (e < n) {
    update_lane_tail(d, e, n, c, clip, coef);
  }
}

// ------------------------------------------------------- micro-step accumulation

// acc += micro (or acc = micro) over a list of tensors, one slice per wave.
__global__ __launch_bounds__(kWave) void accumulate_list_kernel(
    const tm_accum_t* __restrict__ list, int64_t n_list, const tm_chunk_t* __restrict__ chunks,
    uint32_t first_chunk, uint32_t slices_per_chunk, int64_t chunk_elems) {
  tm_chunk_t ck;
  int64_t start;
  slice_of(chunks, first_chunk, slices_per_chunk, chunk_elems, ck, start);
  if (ck.tensor >= n_list) return;
  const tm_accum_t d = list[ck.tensor];
  if (start >= d.numel || !d.micro) return;
  const int64_t end = min(start + kSlice, d.numel);
  const bool vec = aligned16(d.acc) && aligned8(d.micro);
  float* a = reinterpret_cast<float*>(d.acc);
  const uint16_t* m = reinterpret_cast<const uint16_t*>(d.micro);
  if (d.flags & TM_ACCUM_ASSIGN) slice_apply(AssignBf16{a, m, true}, start, end, vec);
  else slice_apply(AccumBf16{a, m, true}, start, end, vec);
}

// Where slice j of chunk c keeps its partial: chunks are padded to whole groups of
// kSliceGroup slots, and within a group the slot of slice j is (j % 8) * 8 + j / 8. Workgroup
// w of a launch runs on XCD w % 8 and covers slice w % slices_per_chunk (a multiple of 8), so
// the 8 partials one XCD writes for a group are contiguous (64 bytes, whole L2 sectors);
// in slice order they would be interleaved with the other XCDs' and every XCD's L2 would
// write back partly written lines (measured 1.023x the algorithmic write bytes).
static_assert((TM_CHUNK_ALIGN / kSlice) % 8 == 0, "slices per chunk must be a multiple of the 8 XCDs");
__device__ __forceinline__ int64_t slice_slot(int64_t c, int64_t j, int64_t slices_per_chunk) {
  const int64_t stride = (slices_per_chunk + kSliceGroup - 1) / kSliceGroup * kSliceGroup;
  const int64_t k = j % kSliceGroup;
  return c * stride + (j - k) + (k % 8) * 8 + k / 8;
}

// The last micro-step, one wave per slice: the accumulation of accumulate_list_kernel, and
// the slice partial of the new accumulator values (the slice order above, whose lane mapping
// follows the accumulator's alignment alone) written to its slice_slot; a slice past its
// tensor's end writes 0.
__global__ __launch_bounds__(kWave) void accumulate_list_sumsq_kernel(
    const tm_accum_t* __restrict__ list, int64_t n_list, const tm_chunk_t* __restrict__ chunks,
    uint32_t first_chunk, uint32_t slices_per_chunk, int64_t chunk_elems, double* __restrict__ slice_partials) {
  const uint32_t local = blockIdx.x / slices_per_chunk;
  const uint32_t sub = blockIdx.x - local * slices_per_chunk;
  const int64_t c = static_cast<int64_t>(first_chunk) + local;
  const tm_chunk_t ck = chunks[c];
  double p = 0.0;
  if (ck.tensor < n_list) {
    const tm_accum_t d = list[ck.tensor];
    const int64_t start = static_cast<int64_t>(ck.chunk) * chunk_elems + static_cast<int64_t>(sub) * kSlice;
    if (start < d.numel) {
      const int64_t end = min(start + kSlice, d.numel);
      float* a = reinterpret_cast<float*>(d.acc);
      const bool vec = aligned16(d.acc);
      if (d.micro) {
        const uint16_t* m = reinterpret_cast<const uint16_t*>(d.micro);
        const bool mvec = aligned8(d.micro);
        p = (d.flags & TM_ACCUM_ASSIGN) ? slice_sumsq(AssignBf16{a, m, mvec}, start, end, vec)
                                        : slice_sumsq(AccumBf16{a, m, mvec}, start, end, vec);
      } else {  // no micro-grad this step: the accumulator only enters the norm
        p = slice_sumsq(ReadF32{a}, start, end, vec);
      }
    }
  }
  if (threadIdx.x == 0) slice_partials[slice_slot(c, sub, slices_per_chunk)] = p;
}

// Block b of the fixed grid of TM_NORM_PARTIALS: the chunk totals of its chunks b, b + G, ...
// from their slice partials, added in chunk order (the slice order above), into partials[b].
__global__ __launch_bounds__(kWave) void slice_reduce_kernel(const double* __restrict__ slice_partials,
                                                             int64_t n_chunks, int64_t slices_per_chunk,
                                                             double* __restrict__ partials) {
  double total = 0.0;
  for (int64_t c = blockIdx.x; c < n_chunks; c += gridDim.x) {
    double lane_acc = 0.0;
    for (int64_t j = threadIdx.x; j < slices_per_chunk; j += kWave)
      lane_acc += slice_partials[slice_slot(c, j, slices_per_chunk)];
    total += slice_wave_sum(lane_acc);
  }
  if (threadIdx.x == 0) partials[blockIdx.x] = total;
}

// ------------------------------------------------------------------- elementwise

// Single-tensor kernels, one slice of kSlice elements per wave; `first` is the slice
// index of the launch's first workgroup (a tensor may need several launches).
__global__ __launch_bounds__(kWave) void accumulate_kernel(float* __restrict__ acc,
                                                           const uint16_t* __restrict__ micro,
                                                           int64_t n, int64_t first) {
  const int64_t start = (first + blockIdx.x) * kSlice;
  const int64_t end = min(start + kSlice, n);
  const bool vec = aligned16(reinterpret_cast<uint64_t>(acc)) &&
                   aligned8(reinterpret_cast<uint64_t>(micro));
  slice_apply(AccumBf16{acc, micro, true}, start, end, vec);
}

// dst (bf16) = RNE(src (fp32)).
struct CastBf16 {
  uint16_t* dst;
  const float* src;
  __device__ __forceinline__ void group(int64_t e) const {
    const f32x4 a = ld<true>(reinterpret_cast<const f32x4*>(src + e));
    u32x2 o;
    o.x = bf16_rne(a.x) | (bf16_rne(a.y) << 16);
    o.y = bf16_rne(a.z) | (bf16_rne(a.w) << 16);
    st<true>(reinterpret_cast<u32x2*>(dst + e), o);
  }
  __device__ __forceinline__ void one(int64_t i) const { dst[i] = static_cast<uint16_t>(bf16_rne(src[i])); }
};

__global__ __launch_bounds__(kWave) void cast_bf16_kernel(uint16_t* __restrict__ dst,
                                                          const float* __restrict__ src, int64_t n,
                                                          int64_t first) {
  const int64_t start = (first + blockIdx.x) * kSlice;
  const int64_t end = min(start + kSlice, n);
  const bool vec = aligned8(reinterpret_cast<uint64_t>(dst)) && aligned16(reinterpret_cast<uint64_t>(src));
  slice_apply(CastBf16{dst, src}, start, end, vec);
}

// The same cast over a list of tensors (param_bf16 = RNE(master) of each record that has a
// working copy), one slice per wave.
__global__ __launch_bounds__(kWave) void cast_bf16_list_kernel(
    const tm_tensor_t* __restrict__ tensors, int64_t n_tensors, const tm_chunk_t* __restrict__ chunks,
    uint32_t first_chunk, uint32_t slices_per_chunk, int64_t chunk_elems) {
  tm_chunk_t ck;
  int64_t start;
  slice_of(chunks, first_chunk, slices_per_chunk, chunk_elems, ck, start);
  if (ck.tensor >= n_tensors) return;
  const tm_tensor_t d = tensors[ck.tensor];
  if (start >= d.numel || !d.param_bf16) return;
  const int64_t end = min(start + kSlice, d.numel);
  const bool vec = aligned8(d.param_bf16) && aligned16(d.master);
  slice_apply(CastBf16{reinterpret_cast<uint16_t*>(d.param_bf16), reinterpret_cast<const float*>(d.master)},
              start, end, vec);
}

// dst = src, 1 KiB per one-wave workgroup (16 bytes a lane, non-temporal), the launch shape of
// the streaming kernels with no cap. The best 1:1 read/write stream measured on MI355X among
// 1, 2 and 4 KiB per wave, with and without occupancy caps (6.72 TB/s over 4 GiB, against
// 4.8 TB/s for the runtime's copy): the ceiling the update's mixed stream is compared with.
__global__ __launch_bounds__(kWave) void stream_copy_kernel(u32x4* __restrict__ dst, const u32x4* __restrict__ src,
                                                            int64_t n_vec, int64_t first) {
  const int64_t i = (first + blockIdx.x) * kWave + threadIdx.x;
  if (i < n_vec) st<true>(dst + i, ld<true>(src + i));
}

// Launches kernel(first, blocks) over `n_slices` one-wave slices in as many launches as the
// 2^32 work-item limit of a launch requires.
template <class F>
int launch_slices(int64_t n_slices, const char* what, F&& launch) {
  for (int64_t first = 0; first < n_slices; first += kMaxSliceBlocks) {
    const int64_t cnt = min(static_cast<int64_t>(kMaxSliceBlocks), n_slices - first);
    launch(first, dim3(static_cast<uint32_t>(cnt)));
    if (int rc = check_launch(what)) return rc;
  }
  return TM_OK;
}

// The same over a chunk table: kernel(first_chunk, slices_per_chunk, blocks), each launch
// covering whole chunks with slices of slice_elems (a divisor of TM_CHUNK_ALIGN).
template <class F>
int launch_chunk_slices(int64_t n_chunks, int64_t chunk_elems, const char* what, F&& launch,
                        int64_t slice_elems = kSlice) {
  const uint32_t spc = static_cast<uint32_t>(chunk_elems / slice_elems);
  const int64_t per = kMaxSliceBlocks / spc;
  for (int64_t first = 0; first < n_chunks; first += per) {
    const int64_t cnt = min(per, n_chunks - first);
    launch(static_cast<uint32_t>(first), spc, dim3(static_cast<uint32_t>(cnt * spc)));
    if (int rc = check_launch(what)) return rc;
  }
  return TM_OK;
}

int check_table(const void* d_tensors, int64_t n_tensors, const void* d_chunks, int64_t n_chunks,
                int64_t chunk_elems, const char* who) {
  if (n_tensors < 0 || n_chunks < 0) return fail(TM_EINVAL, "%s: negative size", who);
  if (n_tensors > 0 && !d_tensors) return fail(TM_EINVAL, "%s: null tensor table", who);
  if (n_chunks > 0 && !d_chunks) return fail(TM_EINVAL, "%s: null chunk table", who);
  if (n_tensors > 0xFFFFFFFFll) return fail(TM_EINVAL, "%s: too many tensors", who);
  // Chunk indices are 32-bit; launches are split to stay under 2^32 work-items each.
  if (n_chunks > 0xFFFFFFFFll)
    return fail(TM_EINVAL, "%s: %lld chunks, at most %lld (use larger chunks)", who,
                (long long)n_chunks, 0xFFFFFFFFll);
  if (chunk_elems <= 0 || chunk_elems % TM_CHUNK_ALIGN != 0 || chunk_elems > (int64_t(1) << 30))
    return fail(TM_EINVAL, "%s: chunk_elems %lld must be a positive multiple of %d, <= 2^30", who,
                (long long)chunk_elems, TM_CHUNK_ALIGN);
  return TM_OK;
}

int check_step_args(const tm_tensor_t* d_tensors, int64_t n_tensors, const tm_chunk_t* d_chunks,
                    int64_t n_chunks, int64_t chunk_elems, const tm_hyper_t* h_groups, int32_t n_groups,
                    const char* who) {
  int rc = check_table(d_tensors, n_tensors, d_chunks, n_chunks, chunk_elems, who);
  if (rc) return rc;
  if (n_groups < 1 || n_groups > TM_MAX_GROUPS || !h_groups)
    return fail(TM_EINVAL, "%s: n_groups %d outside 1..%d", who, n_groups, TM_MAX_GROUPS);
  return TM_OK;
}

// prep (step += 1, per-tensor constants into scal) then the update, stream-ordered.
int launch_step(const tm_tensor_t* d_tensors, int64_t n_tensors, const tm_chunk_t* d_chunks, int64_t n_chunks,
                int64_t chunk_elems, const tm_hyper_t* h_groups, int32_t n_groups, const float* d_coef,
                TensorScal* scal, hipStream_t s) {
  if (n_tensors == 0) return TM_OK;
  HyperArgs hyper;
  memset(&hyper, 0, sizeof(hyper));
  for (int i = 0; i < n_groups; ++i) hyper.g[i] = h_groups[i];
  hyper.n = n_groups;
  hipLaunchKernelGGL(adamw_prep_kernel, dim3(static_cast<uint32_t>((n_tensors + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, s, d_tensors, n_tensors, hyper, scal);
  int rc = check_launch("adamw_prep_kernel");
  if (rc) return rc;
  if (n_chunks == 0) return TM_OK;
  // d_coef == NULL: TM_FLAG_CLIP is ignored (every grad is used unscaled).
  return launch_chunk_slices(n_chunks, chunk_elems, "adamw_update_kernel",
                             [&](uint32_t first, uint32_t spc, dim3 grid) {
                               hipLaunchKernelGGL(adamw_update_kernel, grid, dim3(kWave), kUpdateLds, s, d_tensors,
                                                  n_tensors, d_chunks, first, spc, chunk_elems, scal,
                                                  d_coef);
                             });
}

}  // namespace

// ------------------------------------------------- static scratch of the allocation-free step
//
// tm_adamw_step_noalloc keeps its per-tensor constants (64 bytes a tensor, written by the prep
// kernel and read by the update, so nothing in it needs clearing) in this file-scope device
// array instead of a caller's workspace: TM_NOALLOC_MAX_TENSORS entries, 1 MiB on every GPU the
// library runs on, held until the process ends. Its name is a host-side stand-in, never a
// device address: host code uses only the address hipGetSymbolAddress returns, looked up once
// per device with that device current and kept in g_scratch.
static __device__ __align__(256) TensorScal scratch[TM_NOALLOC_MAX_TENSORS];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
TensorScal* g_scratch[kMaxDevices] = {};

// The device the work of stream s runs on (the current device for the null stream).
int stream_device(hipStream_t s, int* dev) {
  hipError_t e = s ? hipStreamGetDevice(s, dev) : hipGetDevice(dev);
  if (e != hipSuccess) return fail(TM_ELAUNCH, "tm_adamw_step_noalloc: no device for the stream: %s",
                                   hipGetErrorString(e));
  if (*dev < 0 || *dev >= kMaxDevices)
    return fail(TM_EINVAL, "tm_adamw_step_noalloc: device %d beyond the %d supported", *dev, kMaxDevices);
  return TM_OK;
}

int static_scratch(hipStream_t s, TensorScal** out) {
  int dev = -1;
  int rc = stream_device(s, &dev);
  if (rc) return rc;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
    void* ptr = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur >= 0 && cur != dev) {
      const hipError_t back = hipSetDevice(cur);
      if (e == hipSuccess) e = back;
    }
    if (e != hipSuccess || !ptr)
      return fail(TM_ELAUNCH, "tm_adamw_step_noalloc: address of the static scratch on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch[dev] = static_cast<TensorScal*>(ptr);
  }
  *out = g_scratch[dev];
  return TM_OK;
}

}  // namespace

// ======================================================================= C ABI

extern "C" {

int tm_abi_version(void) { return TM_ABI_VERSION; }

const char* tm_last_error(void) { return g_err; }

size_t tm_workspace_bytes(int64_t n_tensors) {
  if (n_tensors < 0) n_tensors = 0;
  return align_up(kPartialBytes, 256) + align_up(sizeof(TensorScal) * n_tensors, 256);
}

int64_t tm_count_chunks(const int64_t* h_numels, int64_t n_tensors, int64_t chunk_elems) {
  if (!h_numels && n_tensors > 0) return fail(TM_EINVAL, "tm_count_chunks: null numels");
  if (chunk_elems <= 0) return fail(TM_EINVAL, "tm_count_chunks: chunk_elems <= 0");
  int64_t total = 0;
  for (int64_t t = 0; t < n_tensors; ++t) {
    if (h_numels[t] < 0) return fail(TM_EINVAL, "tm_count_chunks: negative numel at %lld", (long long)t);
    total += (h_numels[t] + chunk_elems - 1) / chunk_elems;
  }
  return total;
}

int64_t tm_fill_chunks(const int64_t* h_numels, int64_t n_tensors, int64_t chunk_elems,
                       tm_chunk_t* h_out, int64_t cap) {
  const int64_t need = tm_count_chunks(h_numels, n_tensors, chunk_elems);
  if (need < 0) return need;
  if (need > cap || (need > 0 && !h_out))
    return fail(TM_EINVAL, "tm_fill_chunks: need %lld entries, capacity %lld", (long long)need,
                (long long)cap);
  if (n_tensors > 0xFFFFFFFFll) return fail(TM_EINVAL, "tm_fill_chunks: too many tensors");
  int64_t k = 0;
  for (int64_t t = 0; t < n_tensors; ++t) {
    const int64_t nc = (h_numels[t] + chunk_elems - 1) / chunk_elems;
    if (nc > 0xFFFFFFFFll) return fail(TM_EINVAL, "tm_fill_chunks: tensor %lld too large", (long long)t);
    for (int64_t c = 0; c < nc; ++c) {
      h_out[k].tensor = static_cast<uint32_t>(t);
      h_out[k].chunk = static_cast<uint32_t>(c);
      ++k;
    }
  }
  return k;
}

int tm_grad_norm(const tm_tensor_t* d_tensors, int64_t n_tensors, const tm_chunk_t* d_chunks,
                 int64_t n_chunks, int64_t chunk_elems, float max_norm, int clip, void* d_ws,
                 float* d_norm, float* d_coef, void* stream) {
  int rc = check_table(d_tensors, n_tensors, d_chunks, n_chunks, chunk_elems, "tm_grad_norm");
  if (rc) return rc;
  if (!d_ws || !d_norm) return fail(TM_EINVAL, "tm_grad_norm: null workspace or norm output");
  if (clip && !d_coef) return fail(TM_EINVAL, "tm_grad_norm: clip requested with null coef output");
  hipStream_t s = static_cast<hipStream_t>(stream);
  double* partials = static_cast<double*>(d_ws);
  hipLaunchKernelGGL(norm_partials_kernel, dim3(TM_NORM_PARTIALS), dim3(kThreads), 0, s, d_tensors,
                     n_tensors, d_chunks, n_chunks, chunk_elems, partials);
  if ((rc = check_launch("norm_partials_kernel"))) return rc;
  hipLaunchKernelGGL(norm_finalize_kernel, dim3(1), dim3(kThreads), 0, s, partials, max_norm, clip,
                     d_norm, d_coef);
  return check_launch("norm_finalize_kernel");
}

int tm_grad_scale(const tm_tensor_t* d_tensors, int64_t n_tensors, const tm_chunk_t* d_chunks,
                  int64_t n_chunks, int64_t chunk_elems, const float* d_coef, void* stream) {
  int rc = check_table(d_tensors, n_tensors, d_chunks, n_chunks, chunk_elems, "tm_grad_scale");
  if (rc) return rc;
  if (!d_coef) return fail(TM_EINVAL, "tm_grad_scale: null coef");
  hipStream_t s = static_cast<hipStream_t>(stream);
  return launch_chunk_slices(
      n_chunks, chunk_elems, "grad_scale_kernel",
      [&](uint32_t first, uint32_t spc, dim3 grid) {
        hipLaunchKernelGGL(grad_scale_kernel, grid, dim3(kWave), 0, s, d_tensors, n_tensors, d_chunks, first,
                           spc, chunk_elems, d_coef);
      },
      kScaleSlice);
}

int tm_adamw_step(const tm_tensor_t* d_tensors, int64_t n_tensors, const tm_chunk_t* d_chunks,
                  int64_t n_chunks, int64_t chunk_elems, const tm_hyper_t* h_groups,
                  int32_t n_groups, const float* d_coef, void* d_ws, void* stream) {
  int rc = check_step_args(d_tensors, n_tensors, d_chunks, n_chunks, chunk_elems, h_groups, n_groups,
                           "tm_adamw_step");
  if (rc) return rc;
  if (!d_ws) return fail(TM_EINVAL, "tm_adamw_step: null workspace");
  TensorScal* scal =
      reinterpret_cast<TensorScal*>(static_cast<char*>(d_ws) + align_up(kPartialBytes, 256));
  return launch_step(d_tensors, n_tensors, d_chunks, n_chunks, chunk_elems, h_groups, n_groups, d_coef, scal,
                     static_cast<hipStream_t>(stream));
}

int tm_adamw_step_noalloc(const tm_tensor_t* d_tensors, int64_t n_tensors, const tm_chunk_t* d_chunks,
                          int64_t n_chunks, int64_t chunk_elems, const tm_hyper_t* h_groups,
                          int32_t n_groups, const float* d_coef, void* stream) {
  int rc = check_step_args(d_tensors, n_tensors, d_chunks, n_chunks, chunk_elems, h_groups, n_groups,
                           "tm_adamw_step_noalloc");
  if (rc) return rc;
  if (n_tensors > TM_NOALLOC_MAX_TENSORS)
    return fail(TM_EINVAL, "tm_adamw_step_noalloc: %lld tensors, at most %d (its static scratch holds %d)",
                (long long)n_tensors, TM_NOALLOC_MAX_TENSORS, TM_NOALLOC_MAX_TENSORS);
  if (n_tensors == 0) return TM_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  TensorScal* scal = nullptr;
  if ((rc = static_scratch(s, &scal))) return rc;
  return launch_step(d_tensors, n_tensors, d_chunks, n_chunks, chunk_elems, h_groups, n_groups, d_coef, scal, s);
}

size_t tm_accum_norm_workspace_bytes(int64_t n_chunks, int64_t chunk_elems) {
  if (n_chunks < 0 || chunk_elems <= 0) return 0;
  const int64_t spc = chunk_elems / kSlice;
  const int64_t stride = (spc + kSliceGroup - 1) / kSliceGroup * kSliceGroup;  // slice_slot's padding
  return align_up(kPartialBytes, 256) +
         align_up(sizeof(double) * static_cast<size_t>(n_chunks) * static_cast<size_t>(stride), 256);
}

int tm_grad_accumulate_list(const tm_accum_t* d_list, int64_t n_list, const tm_chunk_t* d_chunks,
                            int64_t n_chunks, int64_t chunk_elems, int with_norm, void* d_ws, size_t ws_bytes,
                            float* d_norm, void* stream) {
  int rc = check_table(d_list, n_list, d_chunks, n_chunks, chunk_elems, "tm_grad_accumulate_list");
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (with_norm) {
    if (!d_ws || !d_norm)
      return fail(TM_EINVAL, "tm_grad_accumulate_list: norm requested with null workspace or output");
    const size_t need = tm_accum_norm_workspace_bytes(n_chunks, chunk_elems);
    if (ws_bytes < need)
      return fail(TM_EINVAL, "tm_grad_accumulate_list: workspace of %zu bytes, %zu needed for the norm", ws_bytes,
                  need);
    double* partials = static_cast<double*>(d_ws);
    double* slice_partials = reinterpret_cast<double*>(static_cast<char*>(d_ws) + align_up(kPartialBytes, 256));
    rc = launch_chunk_slices(n_chunks, chunk_elems, "accumulate_list_sumsq_kernel",
                             [&](uint32_t first, uint32_t spc, dim3 grid) {
                               hipLaunchKernelGGL(accumulate_list_sumsq_kernel, grid, dim3(kWave), 0, s, d_list,
                                                  n_list, d_chunks, first, spc, chunk_elems, slice_partials);
                             });
    if (rc) return rc;
    hipLaunchKernelGGL(slice_reduce_kernel, dim3(TM_NORM_PARTIALS), dim3(kWave), 0, s, slice_partials, n_chunks,
                       chunk_elems / kSlice, partials);
    if ((rc = check_launch("slice_reduce_kernel"))) return rc;
    hipLaunchKernelGGL(norm_finalize_kernel, dim3(1), dim3(kThreads), 0, s, partials, 0.0f, 0,
                       d_norm, static_cast<float*>(nullptr));
    return check_launch("norm_finalize_kernel");
  }
  return launch_chunk_slices(n_chunks, chunk_elems, "accumulate_list_kernel",
                             [&](uint32_t first, uint32_t spc, dim3 grid) {
                               hipLaunchKernelGGL(accumulate_list_kernel, grid, dim3(kWave), 0, s, d_list,
                                                  n_list, d_chunks, first, spc, chunk_elems);
                             });
}

int tm_clip_coef(const float* d_norm, float max_norm, float* d_coef, void* stream) {
  if (!d_norm || !d_coef) return fail(TM_EINVAL, "tm_clip_coef: null pointer");
  hipLaunchKernelGGL(clip_coef_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), d_norm,
                     max_norm, d_coef);
  return check_launch("clip_coef_kernel");
}

int tm_grad_accumulate_bf16(float* d_acc, const uint16_t* d_micro, int64_t numel, void* stream) {
  if (numel < 0) return fail(TM_EINVAL, "tm_grad_accumulate_bf16: negative numel");
  if (numel == 0) return TM_OK;
  if (!d_acc || !d_micro) return fail(TM_EINVAL, "tm_grad_accumulate_bf16: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  return launch_slices((numel + kSlice - 1) / kSlice, "accumulate_kernel", [&](int64_t first, dim3 grid) {
    hipLaunchKernelGGL(accumulate_kernel, grid, dim3(kWave), 0, s, d_acc, d_micro, numel, first);
  });
}

int tm_cast_bf16(uint16_t* d_dst, const float* d_src, int64_t numel, void* stream) {
  if (numel < 0) return fail(TM_EINVAL, "tm_cast_bf16: negative numel");
  if (numel == 0) return TM_OK;
  if (!d_dst || !d_src) return fail(TM_EINVAL, "tm_cast_bf16: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  return launch_slices((numel + kSlice - 1) / kSlice, "cast_bf16_kernel", [&](int64_t first, dim3 grid) {
    hipLaunchKernelGGL(cast_bf16_kernel, grid, dim3(kWave), 0, s, d_dst, d_src, numel, first);
  });
}

int tm_stream_copy(void* d_dst, const void* d_src, int64_t nbytes, void* stream) {
  if (nbytes < 0 || nbytes % 16) return fail(TM_EINVAL, "tm_stream_copy: nbytes %lld must be a non-negative multiple of 16",
                                             (long long)nbytes);
  if (nbytes == 0) return TM_OK;
  if (!d_dst || !d_src || ((reinterpret_cast<uint64_t>(d_dst) | reinterpret_cast<uint64_t>(d_src)) & 15u))
    return fail(TM_EINVAL, "tm_stream_copy: null or not 16-byte aligned pointer");
  const uint64_t d0 = reinterpret_cast<uint64_t>(d_dst), s0 = reinterpret_cast<uint64_t>(d_src);
  if (d0 < s0 + static_cast<uint64_t>(nbytes) && s0 < d0 + static_cast<uint64_t>(nbytes))
    return fail(TM_EINVAL, "tm_stream_copy: source and destination overlap");
  const int64_t n_vec = nbytes / 16;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return launch_slices((n_vec + kWave - 1) / kWave, "stream_copy_kernel", [&](int64_t first, dim3 grid) {
    hipLaunchKernelGGL(stream_copy_kernel, grid, dim3(kWave), 0, s, static_cast<u32x4*>(d_dst),
                       static_cast<const u32x4*>(d_src), n_vec, first);
  });
}

int tm_cast_bf16_list(const tm_tensor_t* d_tensors, int64_t n_tensors, const tm_chunk_t* d_chunks,
                      int64_t n_chunks, int64_t chunk_elems, void* stream) {
  int rc = check_table(d_tensors, n_tensors, d_chunks, n_chunks, chunk_elems, "tm_cast_bf16_list");
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return launch_chunk_slices(n_chunks, chunk_elems, "cast_bf16_list_kernel",
                             [&](uint32_t first, uint32_t spc, dim3 grid) {
                               hipLaunchKernelGGL(cast_bf16_list_kernel, grid, dim3(kWave), 0, s, d_tensors,
                                                  n_tensors, d_chunks, first, spc, chunk_elems);
                             });
}

}  // extern "C"
