// tm_ce_gemm.hip -- gfx950 bf16 MFMA GEMM for grad_hidden of the fused linear + cross-entropy.
//
// Per chunk of rows the reference computes grad_h = grad_logits @ W
// (torchure/loss/fused_linear_ce.py:55, a bf16 matmul: fp32 accumulation, bf16 result), with
// grad_logits (rows x V) and W (V x D). For the reference's default chunk of 1024 rows this is
// a long-K GEMM (K = V = 151,936 for the Qwen3 head) with a small output (1024 x 1024): 16
// tiles of 256 x 256, far too few for 256 CUs, and the library GEMM reached about 470 TFLOP/s
// on it. This kernel splits the K range instead:
//   grad_h_gemm_kernel   workgroup (tile, split) computes a 256 x 256 output tile over one
//                        K range with v_mfma_f32_32x32x16_bf16, 8 wave64 (2 x 4, each 128 x 64),
//                        fp32 accumulators, and writes the fp32 partial tile;
//   grad_h_reduce_kernel sums the partials of each element over the splits in a fixed order
//                        (split 0 first) and rounds to bf16 (RNE), so the result does not depend
//                        on scheduling.
// Operands: grad_logits row-major (K contiguous) and W^T (D x V, K contiguous, made by
// transpose_bf16_kernel), both streamed global -> LDS with direct loads (global_load_lds,
// 16 bytes a lane) into a two-stage ring of 64-deep K slices. gfx950's LDS has 64 four-byte
// banks and serves a 16-byte-per-lane read 16 lanes at a time, so the 16 lanes reading 16
// consecutive 128-byte rows must hit 16 different 16-byte bank groups: a row's chunk c sits at
// slot c ^ ((row >> 1) & 7), which gives rows 2j and 2j+1 (one even, one odd: the two halves
// of the banks) the slot pattern c ^ j. (The 32-bank pattern c ^ (row & 7) put rows r and r+8
// on one bank group and doubled the read time; rocprof counted half the LDS cycles as bank
// conflicts.) All the
// workgroups of one split run on one XCD (workgroup w runs on XCD w % 8), so that split's
// K slices of both operands are read from HBM about once and then served from that XCD's L2.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include <mutex>

#include "torchure_amd.h"
#include "tm_internal.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <typename... A>
int gemm_fail(int code, const char* fmt, A... args) {
  return tm_internal_fail(code, fmt, args...);
}

constexpr int kTile = 256;      // output tile edge (rows and columns)
constexpr int kSliceK = 64;     // K depth of one LDS stage (128 bytes of bf16 per row)
constexpr int kStages = 2;
constexpr int kWavesM = 2, kWavesN = 4;
constexpr int kGemmThreads = 64 * kWavesM * kWavesN;
constexpr int kStageBytes = 2 * kTile * kSliceK * 2;  // A and B slices, 64 KB
constexpr int kGemmLds = kStages * kStageBytes;        // 128 KB of the 160 KB per CU
constexpr int kLoadsPerWave = 2 * kTile / 8 / (kWavesM * kWavesN);  // 1 KB load instructions per stage
constexpr int kBlocksM = kTile / kWavesM / 32, kBlocksN = kTile / kWavesN / 32;  // 32x32 blocks per wave

// s_waitcnt immediate that waits for vmcnt <= n only (gfx9 encoding: vmcnt bits 3:0 and
// 15:14; expcnt and lgkmcnt at their maxima, so they are not waited for).
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Output tile and K range of workgroup w in a launch of tiles x splits workgroups (splits a
// multiple of 8): w % 8 is the XCD w runs on; split s = w % 8 + 8 * (w / (8 * tiles)).
__global__ __launch_bounds__(kGemmThreads) void grad_h_gemm_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ Bt, float* __restrict__ partials,
    int rows, int dim, int64_t K, int splits, int iters_per_split) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tiles_n = dim / kTile;
  const int tiles = (rows / kTile) * tiles_n;
  const int w = blockIdx.x;
  const int s = (w % 8) + 8 * (w / (8 * tiles));
  const int tile = (w / 8) % tiles;
  const int m0 = (tile / tiles_n) * kTile, n0 = (tile % tiles_n) * kTile;
  const int total_iters = static_cast<int>(K / kSliceK);
  const int it0 = s * iters_per_split;
  const int it1 = min(it0 + iters_per_split, total_iters);
  const int n_it = it1 > it0 ? it1 - it0 : 0;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / kWavesN, wn = wave % kWavesN;
  const int lrow = lane >> 3, lpos = lane & 7;

  // One stage: kTile rows of A then kTile rows of Bt, 64 bf16 each; load instruction q of the
  // stage fills rows 8q .. 8q+7 (1 KB, lane i -> row 8q + i/8, chunk slot i%8), loading the
  // row's 16-byte chunk (i%8) ^ ((row >> 1) & 7), so that chunk c ends up in slot
  // c ^ ((row >> 1) & 7).
  auto issue = [&](int it, int stage) {
    const int64_t k0 = static_cast<int64_t>(it) * kSliceK;
    uint8_t* base = smem + stage * kStageBytes;
#pragma unroll
    for (int j = 0; j < kLoadsPerWave; ++j) {
      const int q = wave * kLoadsPerWave + j;  // 0 .. 63: A rows for q < 32, Bt rows after
      const int r = (q & 31) * 8 + lrow;
      const int c = lpos ^ ((r >> 1) & 7);
      const uint16_t* src = q < 32 ? A + static_cast<int64_t>(m0 + r) * K : Bt + static_cast<int64_t>(n0 + r) * K;
      __builtin_amdgcn_global_load_lds(
          (const void __attribute__((address_space(1)))*)(src + k0 + c * 8),
          (void __attribute__((address_space(3)))*)(base + q * 1024), 16, 0, 0);
    }
  };

  f32x16 acc[kBlocksM][kBlocksN];
#pragma unroll
  for (int i = 0; i < kBlocksM; ++i)
#pragma unroll
    for (int j = 0; j < kBlocksN; ++j) acc[i][j] = f32x16{};

  if (n_it > 0) issue(it0, 0);
  for (int i = 0; i < n_it; ++i) {
    // This wave's loads of stage i are the only ones in flight (two stages): wait for them,
    // then a bare barrier makes every wave's loads of the stage visible and ensures every wave
    // has consumed its reads of the stage the next issue overwrites (they fed the MFMAs). A
    // __syncthreads() would add a fence that drains every load in flight.
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __builtin_amdgcn_s_barrier();
    if (i + 1 < n_it) issue(it0 + i + 1, (i + 1) & 1);
    const uint8_t* base = smem + (i & 1) * kStageBytes;
#pragma unroll
    for (int kk = 0; kk < kSliceK / 16; ++kk) {
      const int kc = kk * 2 + (lane >> 5);  // this lane's 16-byte chunk of the 128-byte row
      bf16x8 a[kBlocksM], b[kBlocksN];
#pragma unroll
      for (int mi = 0; mi < kBlocksM; ++mi) {
        const int r = wm * (kTile / kWavesM) + mi * 32 + (lane & 31);
        a[mi] = *(const bf16x8*)(base + r * 128 + ((kc ^ ((r >> 1) & 7)) * 16));
      }
#pragma unroll
      for (int ni = 0; ni < kBlocksN; ++ni) {
        const int r = wn * (kTile / kWavesN) + ni * 32 + (lane & 31);
        b[ni] = *(const bf16x8*)(base + kTile * 128 + r * 128 + ((kc ^ ((r >> 1) & 7)) * 16));
      }
#pragma unroll
      for (int mi = 0; mi < kBlocksM; ++mi)
#pragma unroll
        for (int ni = 0; ni < kBlocksN; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[mi], b[ni], acc[mi][ni], 0, 0, 0);
    }
  }
  // D layout of v_mfma_f32_32x32x16_bf16: register r of lane l holds
  // D[8 * (r / 4) + 4 * (l / 32) + r % 4][l % 32].
  float* P = partials + static_cast<int64_t>(s) * rows * dim;
#pragma unroll
  for (int mi = 0; mi < kBlocksM; ++mi)
#pragma unroll
    for (int ni = 0; ni < kBlocksN; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * (kTile / kWavesM) + mi * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
        const int col = n0 + wn * (kTile / kWavesN) + ni * 32 + (lane & 31);
        P[static_cast<int64_t>(row) * dim + col] = acc[mi][ni][r];
      }
}

__device__ __forceinline__ uint32_t rne_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
  return (f != f) ? 0x7FC0u : r;
}

// out[i] = bf16(((P[0][i] + P[1][i]) + P[2][i]) + ...), four elements per thread.
__global__ __launch_bounds__(256) void grad_h_reduce_kernel(const float* __restrict__ partials,
                                                            uint16_t* __restrict__ out, int64_t n, int splits) {
  const int64_t e = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (e >= n) return;
  f32x4 sum = *(const f32x4*)(partials + e);
  for (int s = 1; s < splits; ++s) {
    const f32x4 p = *(const f32x4*)(partials + static_cast<int64_t>(s) * n + e);
    sum.x = sum.x + p.x;
    sum.y = sum.y + p.y;
    sum.z = sum.z + p.z;
    sum.w = sum.w + p.w;
  }
  u32x2 o;
  o.x = rne_bf16(sum.x) | (rne_bf16(sum.y) << 16);
  o.y = rne_bf16(sum.z) | (rne_bf16(sum.w) << 16);
  *(u32x2*)(out + e) = o;
}

// dst (cols x rows) = src (rows x cols)^T, bf16, in 64 x 64 tiles through LDS.
__global__ __launch_bounds__(256) void transpose_bf16_kernel(uint16_t* __restrict__ dst,
                                                             const uint16_t* __restrict__ src, int64_t rows,
                                                             int64_t cols) {
  __shared__ uint16_t t[64][64 + 4];
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64, c0 = static_cast<int64_t>(blockIdx.x) * 64;
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // 64 rows x 16 eight-byte pieces
    const int v = threadIdx.x + 256 * i, r = v >> 4, c = (v & 15) * 4;
    const u32x2 w = *(const u32x2*)(src + (r0 + r) * cols + c0 + c);
    t[r][c] = static_cast<uint16_t>(w.x);
    t[r][c + 1] = static_cast<uint16_t>(w.x >> 16);
    t[r][c + 2] = static_cast<uint16_t>(w.y);
    t[r][c + 3] = static_cast<uint16_t>(w.y >> 16);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // 64 dst rows (src columns) x 16 eight-byte pieces
    const int v = threadIdx.x + 256 * i, c = v >> 4, r = (v & 15) * 4;
    u32x2 w;
    w.x = static_cast<uint32_t>(t[r][c]) | (static_cast<uint32_t>(t[r + 1][c]) << 16);
    w.y = static_cast<uint32_t>(t[r + 2][c]) | (static_cast<uint32_t>(t[r + 3][c]) << 16);
    *(u32x2*)(dst + (c0 + c) * rows + r0 + r) = w;
  }
}

// Splits of the K range: a multiple of 8 (one group of splits per XCD), chosen by a cost model
// of the launch. One 128 KB-LDS workgroup fits a CU, so tiles x S workgroups run in
// ceil(tiles x S / 256) rounds; a workgroup takes about 2 us per 64-deep K slice (256 x 256 x 64
// MFMA work at the kernel's ~1 PFLOP/s over 256 CUs) plus about 8 us to store its 256 KB fp32
// partial tile, and the reduction reads S x rows x dim fp32 partials at about 5 TB/s. The
// model picks S = 16 for the 1024-row Qwen3-0.6B chunk (256 workgroups, one round) and S = 32
// for a 1024-row chunk of a 2560-wide head (40 tiles: 1280 workgroups, five full rounds).
int64_t splits_for(int64_t rows, int64_t vocab, int64_t dim) {
  const int64_t tiles = (rows / kTile) * (dim / kTile);
  const int64_t iters = vocab / kSliceK;
  int64_t best = 8;
  double best_us = 0.0;
  for (int64_t s = 8; s <= 256; s += 8) {
    const int64_t rounds = (tiles * s + 255) / 256;
    const double us = static_cast<double>(rounds) * (2.0 * static_cast<double>((iters + s - 1) / s) + 8.0) +
                      static_cast<double>(s) * static_cast<double>(rows * dim) * 4.0 / 5e6;
    if (s == 8 || us < best_us) {
      best = s;
      best_us = us;
    }
  }
  return best;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The kernel's 128 KB of dynamic LDS exceeds the 64 KB default: the attribute is set once per
// device, with that device current, before the first launch there.
constexpr int kMaxDevices = 64;
std::mutex g_lds_mu;
bool g_lds_set[kMaxDevices] = {};

hipError_t allow_lds(hipStream_t stream) {
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_lds_mu);
  if (g_lds_set[dev]) return hipSuccess;
  int cur = -1;
  e = hipGetDevice(&cur);
  if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
  if (e == hipSuccess)
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(grad_h_gemm_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kGemmLds);
  if (cur >= 0 && cur != dev) {
    const hipError_t back = hipSetDevice(cur);
    if (e == hipSuccess) e = back;
  }
  if (e == hipSuccess) g_lds_set[dev] = true;
  return e;
}

}  // namespace

extern "C" {

size_t tm_ce_grad_h_workspace_bytes(int64_t rows, int64_t vocab, int64_t dim) {
  if (rows <= 0 || dim <= 0 || vocab <= 0 || rows % kTile || dim % kTile || vocab % kSliceK) return 0;
  return static_cast<size_t>(splits_for(rows, vocab, dim)) * rows * dim * sizeof(float);
}

int tm_ce_grad_h_bf16(uint16_t* d_grad_h, const uint16_t* d_grad_logits, const uint16_t* d_wt, int64_t rows,
                      int64_t vocab, int64_t dim, void* d_ws, size_t ws_bytes, void* stream) {
  if (rows <= 0 || dim <= 0 || vocab <= 0 || rows % kTile || dim % kTile || vocab % kSliceK)
    return gemm_fail(TM_EINVAL,
                     "tm_ce_grad_h_bf16: rows %lld and dim %lld must be positive multiples of %d, vocab %lld "
                     "of %d", (long long)rows, (long long)dim, kTile, (long long)vocab, kSliceK);
  if (rows > (1 << 20) || dim > (1 << 16))
    return gemm_fail(TM_EINVAL, "tm_ce_grad_h_bf16: rows %lld or dim %lld too large", (long long)rows,
                     (long long)dim);
  if (!d_grad_h || !d_grad_logits || !d_wt || !d_ws)
    return gemm_fail(TM_EINVAL, "tm_ce_grad_h_bf16: null pointer");
  if (!aligned16(d_grad_h) || !aligned16(d_grad_logits) || !aligned16(d_wt) || !aligned16(d_ws))
    return gemm_fail(TM_EINVAL, "tm_ce_grad_h_bf16: pointers must be 16-byte aligned");
  if (ws_bytes < tm_ce_grad_h_workspace_bytes(rows, vocab, dim))
    return gemm_fail(TM_EINVAL, "tm_ce_grad_h_bf16: workspace of %zu bytes, %zu needed", ws_bytes,
                     tm_ce_grad_h_workspace_bytes(rows, vocab, dim));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const hipError_t lds = allow_lds(s);
  if (lds != hipSuccess)
    return gemm_fail(TM_ELAUNCH, "tm_ce_grad_h_bf16: LDS attribute: %s", hipGetErrorString(lds));
  const int64_t splits = splits_for(rows, vocab, dim);
  const int64_t tiles = (rows / kTile) * (dim / kTile);
  const int64_t total_iters = vocab / kSliceK;
  const int64_t per = (total_iters + splits - 1) / splits;
  float* partials = static_cast<float*>(d_ws);
  hipLaunchKernelGGL(grad_h_gemm_kernel, dim3(static_cast<uint32_t>(tiles * splits)), dim3(kGemmThreads),
                     kGemmLds, s, d_grad_logits, d_wt, partials, static_cast<int>(rows), static_cast<int>(dim),
                     vocab, static_cast<int>(splits), static_cast<int>(per));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return gemm_fail(TM_ELAUNCH, "grad_h_gemm_kernel: launch failed: %s", hipGetErrorString(e));
  const int64_t n = rows * dim;
  hipLaunchKernelGGL(grad_h_reduce_kernel, dim3(static_cast<uint32_t>((n / 4 + 255) / 256)), dim3(256), 0, s,
                     partials, d_grad_h, n, static_cast<int>(splits));
  e = hipGetLastError();
  if (e != hipSuccess) return gemm_fail(TM_ELAUNCH, "grad_h_reduce_kernel: launch failed: %s", hipGetErrorString(e));
  return TM_OK;
}

int tm_ce_transpose_bf16(uint16_t* d_dst, const uint16_t* d_src, int64_t rows, int64_t cols, void* stream) {
  if (rows <= 0 || cols <= 0 || rows % 64 || cols % 64)
    return gemm_fail(TM_EINVAL, "tm_ce_transpose_bf16: rows %lld and cols %lld must be positive multiples of 64",
                     (long long)rows, (long long)cols);
  if (rows / 64 > 65535 || cols / 64 > 0x7FFFFFFF)
    return gemm_fail(TM_EINVAL, "tm_ce_transpose_bf16: %lld rows is too many", (long long)rows);
  if (!d_dst || !d_src || (reinterpret_cast<uintptr_t>(d_dst) & 7u) || (reinterpret_cast<uintptr_t>(d_src) & 7u))
    return gemm_fail(TM_EINVAL, "tm_ce_transpose_bf16: null or not 8-byte aligned pointer");
  hipLaunchKernelGGL(transpose_bf16_kernel, dim3(static_cast<uint32_t>(cols / 64), static_cast<uint32_t>(rows / 64)),
                     dim3(256), 0, static_cast<hipStream_t>(stream), d_dst, d_src, rows, cols);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return gemm_fail(TM_ELAUNCH, "transpose_bf16_kernel: launch failed: %s", hipGetErrorString(e));
  return TM_OK;
}

}  // extern "C"
