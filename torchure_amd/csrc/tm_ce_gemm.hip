// tm_ce_gemm.hip -- gfx950 bf16 MFMA GEMMs of the fused linear + cross-entropy, per chunk of rows
// (torchure/loss/fused_linear_ce.py:38,52,57: bf16 matmuls, fp32 accumulation, bf16 results):
//   logits_ring_kernel   logits = h W^T         (rows x V, K = D), persistent, for dim a multiple
//                        of 128 (>= 256) and vocab a multiple of 8; logits_gemm_kernel otherwise
//   grad_h_gemm_kernel   grad_h = grad_logits W (rows x D, K = V), split over K, reading W as it
//                        is stored (V x D), with
//   grad_h_reduce_kernel summing the fp32 partials of each element over the splits in a fixed
//                        order (split 0 first) and rounding once to bf16 (RNE), so the result
//                        does not depend on scheduling
//   grad_w_ring_kernel   grad_W = grad_logits^T h (V x D, K = rows), persistent, for rows a
//                        multiple of 128 (>= 256); grad_w_gemm_kernel otherwise
//
// All three are 256 x 256 output tiles per workgroup on v_mfma_f32_32x32x16_bf16 with fp32
// accumulation: the ring kernels and grad_h_gemm_kernel on 8 wave64, two a SIMD (each 128 x 64,
// 128 accumulators), so that one wave's MFMAs run while the other waits; the one-tile kernels on
// 4 wave64 (each 128 x 128, 256 accumulators in the AGPRs). Every element sees the same MFMA
// sequence in the ring and one-tile kernels. Operands stream
// global -> LDS with direct loads (global_load_lds, 16 bytes a lane) into two 64 KB stages of
// 64-deep K slices. gfx950's LDS has 64 four-byte banks and serves a 16-byte-per-lane read 16
// lanes at a time, so the 16 lanes reading 16 consecutive 128-byte rows must hit 16 different
// 16-byte bank groups: a row's chunk c sits at slot c ^ ((row >> 1) & 7), which gives rows 2j and
// 2j+1 (one even, one odd: the two halves of the banks) the slot pattern c ^ j. (The 32-bank
// pattern c ^ (row & 7) put rows r and r+8 on one bank group and doubled the read time.)
// Workgroup w runs on XCD w % 8; each XCD takes a contiguous range of tiles (or of split-tile
// pairs), so the operand panels its 32 CUs share are read from HBM about once and then served
// from that XCD's L2.
//
// For the reference's default chunk of 1024 rows, grad_h is a long-K GEMM (K = V = 151,936 for
// the Qwen3 head) with a small output (1024 x 1024): 16 tiles for 256 CUs, which the library GEMM
// ran at about 450 TFLOP/s. Splitting K gives every CU a (split, tile) pair.

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
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

template <typename... A>
int gemm_fail(int code, const char* fmt, A... args) {
  return tm_internal_fail(code, fmt, args...);
}

constexpr int kTile = 256;      // output tile edge (rows and columns)
constexpr int kSliceK = 64;     // K depth of one LDS stage (128 bytes of bf16 per row)

// s_waitcnt immediate that waits for vmcnt <= n only (gfx9 encoding: vmcnt bits 3:0 and
// 15:14; expcnt and lgkmcnt at their maxima, so they are not waited for).
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

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

// ------------------------------------------------------------------ logits = hidden @ W^T
//
// fused_linear_ce.py:38 `logits = h @ w.t()` per chunk: C (rows x vocab) = A (rows x dim) times
// B (vocab x dim) transposed, both operands K-contiguous (K = dim), bf16 in and out, fp32
// accumulation. A 256 x 256 output tile per workgroup of 4 wave64 (2 x 2), each wave 128 x 128
// with 256 fp32 accumulators (the AGPRs) on v_mfma_f32_32x32x16_bf16. Operands stream
// global -> LDS (global_load_lds, 16 bytes a lane, 1 KB = 8 rows of a 64-deep K slice per
// instruction) into two 64 KB stages whose 128-byte rows hold their 16-byte chunks at slot
// c ^ ((row >> 1) & 7). Schedule per 64-deep stage (4 K16 steps), in nt_mainloop below:
//   - the next step's 8 fragments (16-byte LDS reads, inline asm) are issued one per two MFMAs
//     of the current step, so the reads run under the MFMAs; sched_barrier pins that order and
//     an `s_waitcnt lgkmcnt(0)` that names the fragments as operands keeps every MFMA behind
//     the wait for its data;
//   - the stage barrier sits at the start of the last K16 step: after it, that step's MFMAs
//     run while the next stage's first fragments are read and the 16 loads of the stage after
//     next are issued into the buffer just finished. No step waits on LDS right after a barrier.
// Operand roles are swapped (the MFMA's first operand is the weight tile), so a lane holds 4
// consecutive output columns of one row; the tile is converted to bf16 (RNE, v_cvt_pk_bf16_f32)
// into LDS rows of 256 B (+16 B pad) and written back in whole rows, 16 bytes a lane: writing
// 8-byte pieces of 32 rows per instruction straight from the accumulators made the L2 take
// 16-byte partial-line writes, twice as many L2 requests as the operand reads, and cost 12%.
// Rows past `rows` and columns past `vocab` load a clamped (valid) row and are not stored.
// Tile order: workgroup w runs on XCD w % 8, which takes a contiguous range of tile positions;
// within it, groups of gm x gn tiles (gm * gn = 32, one per CU of the XCD) run together so that
// their operand panels are read from HBM about once per group and served from that XCD's L2.

constexpr int kLgTile = 256;                                    // output tile edge
constexpr int kLgStage = 2 * kLgTile * kSliceK * 2;             // 64 KB: A and B slices
constexpr int kLgPitch = 272;                                   // output staging row pitch
constexpr int kLgLds = 4 * 128 * kLgPitch > 2 * kLgStage ? 4 * 128 * kLgPitch : 2 * kLgStage;  // 139,264 B

// Tile of position p: n-blocks of gn tile columns; inside each, m-blocks of gm tile rows, a
// block's gm x gn tiles consecutive in p.
__device__ __forceinline__ void lg_tile_of(int p, int tiles_m, int tiles_n, int gm, int gn, int& tm, int& tn) {
  const int per_nb = tiles_m * gn;
  const int nb = p / per_nb, rem = p - nb * per_nb;
  const int gn_eff = min(gn, tiles_n - nb * gn);
  const int mb = rem / (gm * gn_eff), rem2 = rem - mb * gm * gn_eff;
  tm = mb * gm + rem2 / gn_eff;
  tn = nb * gn + rem2 % gn_eff;
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two floats -> packed bf16, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const bf16x2 h = __builtin_convertvector(f32x2{a, b}, bf16x2);
  return __builtin_bit_cast(uint32_t, h);
}

template <bool kN, bool kN2>
struct LgFlags {
  static constexpr bool kNextV = kN, kNext2V = kN2;
};

// Main loop of logits_gemm_kernel (both operands K-contiguous): acc[n block][m block] of a
// 256 x 256 tile, rows m0.. of A and n0.. of B (`ld` elements apart, rows past M or N clamped to
// the last), over n_it 64-deep K slices from element k0. 4 waves, wave (wm, wn) = 128 x 128.
__device__ __forceinline__ void nt_mainloop(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                                            int64_t ld, int m0, int n0, int M, int N, int64_t k0, int n_it,
                                            uint8_t* smem, f32x16 (&acc)[4][4]) {
  const int lane = threadIdx.x & 63;
  // wave-uniform in a scalar register, so each load's LDS destination (M0) is scalar arithmetic
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // Load j of this wave fills LDS rows 8 q .. 8 q + 7 of [A tile; B tile], q = 16 wave + j; the
  // lane loads 16-byte chunk (lane % 8) ^ ((row >> 1) & 7) of row 8 q + lane / 8 into slot lane % 8.
  const uint16_t* src[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int q = wave * 16 + j;
    const int r = (q % 32) * 8 + lane / 8;
    const int c = (lane % 8) ^ ((r >> 1) & 7);
    src[j] = (q < 32 ? A + static_cast<int64_t>(min(m0 + r, M - 1)) * ld
                     : B + static_cast<int64_t>(min(n0 + r, N - 1)) * ld) + k0 + c * 8;
  }
  auto load = [&](int it, int stage, int j) {
    __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)(src[j] + it * kSliceK),
                                     (void __attribute__((address_space(3)))*)(smem + stage * kLgStage + (wave * 16 + j) * 1024),
                                     16, 0, 0);
  };
  // Fragment reads: lane reads row R0 + lane % 32 (R0 a multiple of 32), chunk 2 kk + lane / 32,
  // at slot (2 kk) ^ tx with tx = (lane / 32) ^ ((lane >> 1) & 7).
  const int tx = (lane >> 5) ^ ((lane >> 1) & 7);
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem)) + (lane & 31) * 128;
  uint32_t vk[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) vk[kk] = lds0 + (((2 * kk) ^ tx) * 16);
  const uint32_t offA = wm * 128 * 128, offB = kLgTile * 128 + wn * 128 * 128;

#define TM_RD(dst, base, imm) asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(dst) : "v"(base), "i"(imm))
#define TM_WAIT8(f)                                                                                       \
  asm volatile("s_waitcnt lgkmcnt(0)"                                                                   \
               : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]), "+v"(f[6]), "+v"(f[7]))
  // fragment g: g < 4 -> B (n) block g, g >= 4 -> A (m) block g - 4
  bf16x8 f0[8], f1[8];
#pragma unroll
  for (int j = 0; j < 16; ++j) load(0, 0, j);
  if (n_it > 1) {
#pragma unroll
    for (int j = 0; j < 16; ++j) load(1, 1, j);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(16));
  } else {
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  }
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int g = 0; g < 8; ++g) TM_RD(f0[g], vk[0] + (g < 4 ? offB : offA), (g % 4) * 32 * 128);
  TM_WAIT8(f0);
  __builtin_amdgcn_sched_barrier(0);

  auto stage = [&](int i, auto step) {
    constexpr bool kNext = decltype(step)::kNextV, kNext2 = decltype(step)::kNext2V;
    const int s = i & 1;
    const uint32_t soff = s * kLgStage, noff = (s ^ 1) * kLgStage;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      bf16x8* cur = (kk & 1) ? f1 : f0;
      bf16x8* nxt = (kk & 1) ? f0 : f1;
      if (kk == 3 && kNext) {
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // this wave's loads of stage i + 1 are in LDS
        __builtin_amdgcn_s_barrier();               // every wave's; and stage i's reads are done
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        if (kk < 3) {
          TM_RD(nxt[g], vk[kk + 1] + soff + (g < 4 ? offB : offA), (g % 4) * 32 * 128);
        } else if (kNext) {
          TM_RD(nxt[g], vk[0] + noff + (g < 4 ? offB : offA), (g % 4) * 32 * 128);
        }
        if (kk == 3 && kNext2) {
          load(i + 2, s, 2 * g);
          load(i + 2, s, 2 * g + 1);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int idx = 2 * g + h, ii = idx / 4, jj = idx % 4;
          acc[ii][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur[ii], cur[4 + jj], acc[ii][jj], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (kk < 3 || kNext) {
        TM_WAIT8(nxt);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  int i = 0;
  for (; i + 2 < n_it; ++i) stage(i, LgFlags<true, true>{});
  if (i + 1 < n_it) stage(i++, LgFlags<true, false>{});
  if (i < n_it) stage(i, LgFlags<false, false>{});
#undef TM_RD
#undef TM_WAIT8
}

__global__ __launch_bounds__(256) void logits_gemm_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                                                          uint16_t* __restrict__ C, int M, int N, int K, int tiles_m,
                                                          int tiles_n, int gm, int gn) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int T = tiles_m * tiles_n;
  const int t8 = (T + 7) / 8;
  const int p = (blockIdx.x % 8) * t8 + blockIdx.x / 8;  // XCD blockIdx % 8 takes positions [x t8, (x+1) t8)
  if (p >= T) return;
  int tm, tn;
  lg_tile_of(p, tiles_m, tiles_n, gm, gn, tm, tn);
  const int m0 = tm * kLgTile, n0 = tn * kLgTile;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  f32x16 acc[4][4];  // [n block][m block]
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};
  nt_mainloop(A, B, K, m0, n0, M, N, 0, K / kSliceK, smem, acc);

  // D[n][m] of a 32 x 32 block: register r of lane l holds n = 8 (r / 4) + 4 (l / 32) + r % 4,
  // m = l % 32. Each wave stages its 128 x 128 bf16 tile in LDS, then writes whole rows.
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_s_barrier();  // every wave is done reading the operand stages
  uint8_t* tile = smem + wave * 128 * kLgPitch;
#pragma unroll
  for (int ii = 0; ii < 4; ++ii)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int mr = jj * 32 + (lane & 31), nc = ii * 32 + 8 * q + 4 * (lane >> 5);
        u32x2 o;
        o.x = pack_bf16x2(acc[ii][jj][4 * q], acc[ii][jj][4 * q + 1]);
        o.y = pack_bf16x2(acc[ii][jj][4 * q + 2], acc[ii][jj][4 * q + 3]);
        *(u32x2*)(tile + mr * kLgPitch + nc * 2) = o;
      }
  __builtin_amdgcn_s_waitcnt(0);  // this wave reads back only its own rows
  const int mb = m0 + wm * 128, nb = n0 + wn * 128;
  const bool vec = (N & 7) == 0;
#pragma unroll 4
  for (int it = 0; it < 32; ++it) {
    const int mr = it * 4 + (lane >> 4), ch = lane & 15;
    const int m = mb + mr, n = nb + ch * 8;
    if (m >= M) continue;
    const u32x4 v = *(const u32x4*)(tile + mr * kLgPitch + ch * 16);
    uint16_t* dst = C + static_cast<int64_t>(m) * N + n;
    if (vec && n + 8 <= N) {
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(dst));  // streamed out: keep L2 for operands
    } else {
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
      for (int e = 0; e < 8 && n + e < N; ++e) dst[e] = static_cast<uint16_t>(w[e / 2] >> (16 * (e & 1)));
    }
  }
}

// ------------------------------------------------ logits, persistent: one workgroup per CU
//
// The same product, tiles, fragments and summation order as logits_gemm_kernel (bit-identical
// results), for the shapes the Qwen heads have (dim a multiple of 128 and at least 256, vocab a
// multiple of 8, operands under 4 GiB). With K = dim short (16 slices at dim 1024), a tile's
// fill (its first two stages' loads) and its epilogue (its accumulators converted to bf16 and
// written) were a large share of a tile's time; here both overlap the neighbouring tiles' MFMAs:
//   - workgroup c of XCD x (blockIdx = 8 c + x) runs tile positions x t8 + c, + W, + 2W, ...
//     (W workgroups per XCD), so the 32 tiles an XCD runs at a time are the same groups of
//     tiles as in logits_gemm_kernel;
//   - the operand stages form one ring across tiles: the next tile's stages 0 and 1 are loaded
//     during the current tile's last two stages (the tile after the last is the last again, a
//     harmless reload drained before exit);
//   - 8 waves, two a SIMD: wave (wm, wn) = (w / 4, w % 4) computes rows wm * 128 .. +127 and
//     columns wn * 64 .. +63 of the tile, 4 m blocks x 2 n blocks of 32 x 32 (128 accumulators,
//     in VGPRs); while one wave of a SIMD waits for LDS, its loads, the stage barrier or its
//     stores, the other's MFMAs run (measured on MI355X: 4-12% faster than one wave a SIMD with
//     128 x 128 each, the same bits). Per K16 step a wave reads 6 fragments and issues 8 MFMAs;
//     waves 0-3 load the hidden rows, waves 4-7 the weight rows, 8 loads a stage each;
//   - the finished tile's accumulators leave during the next tile's first K16 step: block
//     (ii, jj) is converted to bf16 (RNE) just before that step's MFMA on it, which restarts
//     its accumulation from zero; the 2 blocks of an m block (32 rows x the wave's 64 columns)
//     go to this wave's 4 KB of LDS past the two stages (128-byte rows, chunk c of row r at slot
//     c ^ ((r >> 1) & 7)) and are written back as 128-byte row pieces, 16 bytes a lane; the
//     last tile's output goes the same way after the loop.
// LDS: two 64 KB stages + 8 x 4 KB = 160 KB, the whole of a CU's. Operand addresses are 32-bit
// byte offsets from the operand's base (scalar), one per load.

constexpr int kRgLds = 2 * kLgStage + 8 * 4096;  // 163,840 B

template <bool kN2, bool kPre, bool kFirst, bool kEpi>
struct RgFlags {
  static constexpr bool kNext2V = kN2, kPreV = kPre, kFirstV = kFirst, kEpiV = kEpi;
};

template <bool kV>
struct RgBool {
  static constexpr bool value = kV;
};

__global__ __launch_bounds__(512) void logits_ring_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                                                          uint16_t* __restrict__ C, int M, int N, int K, int tiles_m,
                                                          int tiles_n, int gm, int gn, int wpx) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int T = tiles_m * tiles_n;
  const int t8 = (T + 7) / 8;
  const int x = blockIdx.x % 8;
  const int pend = min((x + 1) * t8, T);
  int p = x * t8 + static_cast<int>(blockIdx.x / 8);
  if (p >= pend) return;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int n_it = K / kSliceK;  // even, >= 4

  // Waves 0-3 load the A rows of the tile, waves 4-7 the B rows; load j of wave w fills rows
  // 64 (w % 4) + 8 j + lane / 8 of its operand, the lane's chunk (lane % 8) ^ (lane / 16) ^ (4 (j % 2)).
  const char* opnd = reinterpret_cast<const char*>(wave < 4 ? A : B);
  const int lim = (wave < 4 ? M : N) - 1;
  uint32_t soff[8];
  int lrow = lane / 8;
  uint32_t lc16 = static_cast<uint32_t>(((lane % 8) ^ (lane / 16)) * 16);
  auto set_src = [&](int m0, int n0) {
    asm volatile("" : "+v"(lrow), "+v"(lc16));
    const int r0 = (wave < 4 ? m0 : n0) + (wave % 4) * 64;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      soff[j] = static_cast<uint32_t>(min(r0 + 8 * j + lrow, lim)) * static_cast<uint32_t>(2 * K) +
                (lc16 ^ ((j & 1) * 64));
  };
  auto load = [&](int it, int stage, int j) {
    __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)(opnd + (soff[j] + it * 128u)),
                                     (void __attribute__((address_space(3)))*)(smem + stage * kLgStage + (wave * 8 + j) * 1024),
                                     16, 0, 0);
  };
  const int tx = (lane >> 5) ^ ((lane >> 1) & 7);
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem)) + (lane & 31) * 128;
  uint32_t vk[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) vk[kk] = lds0 + (((2 * kk) ^ tx) * 16);
  const uint32_t offA = wm * 128 * 128, offB = kLgTile * 128 + wn * 64 * 128;

  // Output staging, this wave's 4 KB: row r (of an m block's 32) at 128 r, chunk c at slot
  // c ^ ((r >> 1) & 7). A lane writes row lane % 32, half lane / 32 of chunk c; it reads back chunk
  // lane % 8 of row 8 it + lane / 8.
  const uint32_t ebo = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem)) + 2 * kLgStage + wave * 4096;
  const int wr = lane & 31;
  uint32_t wa = ebo + wr * 128 + (lane >> 5) * 8;
  const uint32_t wsw = static_cast<uint32_t>((wr >> 1) & 7);
  uint32_t ra[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int r = k * 8 + (lane >> 3);
    ra[k] = ebo + r * 128 + (((lane & 7) ^ ((r >> 1) & 7)) << 4);
  }
  uint32_t sl = static_cast<uint32_t>(((lane >> 3) * N + (lane & 7) * 8) * 2);  // byte offset of the lane's store

#define TM_RD(dst, base, imm) asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(dst) : "v"(base), "i"(imm))
#define TM_WAIT6(f) \
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]))
  // fragment g: g < 2 -> B (n) block g, g >= 2 -> A (m) block g - 2
  bf16x8 f0[6], f1[6];
  f32x16 acc[2][4];  // [n block][m block]
  int pm0 = 0, pn0 = 0;

  auto epi_block = [&](int ii, int jj, bool mfma, bf16x8* cur) {
    asm volatile("" : "+v"(acc[ii][jj]));
    u32x2 o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      o[q].x = pack_bf16x2(acc[ii][jj][4 * q], acc[ii][jj][4 * q + 1]);
      o[q].y = pack_bf16x2(acc[ii][jj][4 * q + 2], acc[ii][jj][4 * q + 3]);
    }
    if (mfma) {
      asm volatile("" : "+v"(cur[ii]) : "v"(o[0]), "v"(o[1]), "v"(o[2]), "v"(o[3]));
      acc[ii][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur[ii], cur[2 + jj], f32x16{}, 0, 0, 0);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t a = wa + (((static_cast<uint32_t>(ii * 4 + q)) ^ wsw) << 4);
      asm volatile("ds_write_b64 %0, %1" ::"v"(a), "v"(o[q]) : "memory");
    }
  };
  auto epi_store = [&](int jj) {
    u32x4 v[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) asm volatile("ds_read_b128 %0, %1" : "=v"(v[it]) : "v"(ra[it]));
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]));
    const int rows_left = M - (pm0 + wm * 128 + jj * 32), cols_left = N - (pn0 + wn * 64);
    char* qb = reinterpret_cast<char*>(C) + (static_cast<int64_t>(pm0 + wm * 128 + jj * 32) * N + pn0 + wn * 64) * 2;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      if (it * 8 + (lane >> 3) < rows_left && (lane & 7) * 8 < cols_left)
        __builtin_nontemporal_store(v[it], reinterpret_cast<u32x4*>(qb + (sl + static_cast<uint32_t>(it * 8 * N * 2))));
    }
  };

  int tm, tn;
  lg_tile_of(p, tiles_m, tiles_n, gm, gn, tm, tn);
  int m0 = tm * kLgTile, n0 = tn * kLgTile;
  set_src(m0, n0);
#pragma unroll
  for (int j = 0; j < 8; ++j) load(0, 0, j);
#pragma unroll
  for (int j = 0; j < 8; ++j) load(1, 1, j);
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(8));
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int g = 0; g < 6; ++g) TM_RD(f0[g], vk[0] + (g < 2 ? offB : offA), (g < 2 ? g : g - 2) * 32 * 128);
  TM_WAIT6(f0);
  __builtin_amdgcn_sched_barrier(0);

  int pn = p, m0n = m0, n0n = n0;
  bool has_next = false;
  auto tile = [&](auto epi_first) {
    constexpr bool kEpiFirst = decltype(epi_first)::value;
    asm volatile("" : "+v"(wa), "+v"(ra[0]), "+v"(ra[1]), "+v"(ra[2]), "+v"(ra[3]), "+v"(sl));
    pn = p + wpx;
    has_next = pn < pend;
    int tmn, tnn;
    lg_tile_of(has_next ? pn : p, tiles_m, tiles_n, gm, gn, tmn, tnn);
    m0n = tmn * kLgTile;
    n0n = tnn * kLgTile;

    auto stage = [&](int i, auto step) {
      constexpr bool kNext2 = decltype(step)::kNext2V, kPre = decltype(step)::kPreV;
      constexpr bool kFirst = decltype(step)::kFirstV, kEpi = decltype(step)::kEpiV;
      const int s = i & 1;
      const uint32_t soff_s = s * kLgStage, noff = (s ^ 1) * kLgStage;
      if (kPre) {
        set_src(m0n, n0n);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        bf16x8* cur = (kk & 1) ? f1 : f0;
        bf16x8* nxt = (kk & 1) ? f0 : f1;
        if (kEpi && kk == 0) {  // first K16 step, with the previous tile's output
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
            for (int ii = 0; ii < 2; ++ii) {
              const int g = jj * 2 + ii;
              if (g < 6) TM_RD(nxt[g], vk[1] + soff_s + (g < 2 ? offB : offA), (g < 2 ? g : g - 2) * 32 * 128);
              epi_block(ii, jj, true, cur);
              __builtin_amdgcn_sched_barrier(0);
            }
            epi_store(jj);
            __builtin_amdgcn_sched_barrier(0);
          }
          TM_WAIT6(nxt);
          __builtin_amdgcn_sched_barrier(0);
          continue;
        }
        if (kk == 3) {
          __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
          __builtin_amdgcn_s_barrier();
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          if (g < 6) {
            if (kk < 3) {
              TM_RD(nxt[g], vk[kk + 1] + soff_s + (g < 2 ? offB : offA), (g < 2 ? g : g - 2) * 32 * 128);
            } else {
              TM_RD(nxt[g], vk[0] + noff + (g < 2 ? offB : offA), (g < 2 ? g : g - 2) * 32 * 128);
            }
          }
          if (kk == 3 && kNext2) {
            const int it2 = i + 2 >= n_it ? i + 2 - n_it : i + 2;
            load(it2, s, g);
          }
          const int jj = g / 2, ii = g % 2;
          if (kFirst && kk == 0)
            acc[ii][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur[ii], cur[2 + jj], f32x16{}, 0, 0, 0);
          else
            acc[ii][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur[ii], cur[2 + jj], acc[ii][jj], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
        TM_WAIT6(nxt);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    stage(0, RgFlags<true, false, true, kEpiFirst>{});
    for (int i = 1; i < n_it - 2; ++i) stage(i, RgFlags<true, false, false, false>{});
    stage(n_it - 2, RgFlags<true, true, false, false>{});
    stage(n_it - 1, RgFlags<true, false, false, false>{});
    pm0 = m0;
    pn0 = n0;
  };
  tile(RgBool<false>{});
  while (has_next) {
    p = pn;
    m0 = m0n;
    n0 = n0n;
    __builtin_amdgcn_sched_barrier(0);
    tile(RgBool<true>{});
  }
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) epi_block(ii, jj, false, f0);
    epi_store(jj);
  }
  __builtin_amdgcn_s_waitcnt(0);
#undef TM_RD
#undef TM_WAIT6
}

// The ring kernel's preconditions: K slices in an even number >= 4, whole 8-column store groups,
// 32-bit operand offsets and store offsets.
bool logits_ring_fits(int64_t rows, int64_t vocab, int64_t dim) {
  return dim % 128 == 0 && dim >= 256 && vocab % 8 == 0 && rows * dim * 2 < (int64_t(1) << 32) &&
         vocab * dim * 2 < (int64_t(1) << 32) && 32 * vocab * 2 < (int64_t(1) << 32);
}

// ------------------------------------------------- grad_h = grad_logits @ W, K split over workgroups
//
// fused_linear_ce.py:52 `grad_h = grad_logits @ w` per chunk: C (rows x dim) = G (rows x V) times
// W (V x dim), K = V. K is long and the output small (16 tiles for a 1024-row chunk at dim
// 1024), so workgroup (split, tile) computes one 256 x 256 tile over one range of K slices and
// writes its fp32 partial tile (straight from the accumulators, 16 bytes a lane: 4 consecutive
// columns of one row; a split with no K slices writes zeros); grad_h_reduce_kernel adds the
// partials. Pair p = split x tiles + tile; workgroup w runs on XCD w % 8, which takes pairs
// [x p8, (x+1) p8): the workgroups of an XCD share a split's K range of both operands in its L2.
// A stage holds G's 256 rows x 64 K as 128-byte rows (the logits GEMM's layout and fragment
// reads) and W's 64 K rows x 256 columns as 512-byte rows (grad_W's layout for its K-major
// operand, fragments from two ds_read_b64_tr_b16), so W is read as it is stored: no transposed
// copy. 8 waves, two a SIMD, wave (wm, wn) = (w / 4, w % 4) computing rows wm * 128 .. +127 and
// columns wn * 64 .. +63 (4 x 2 blocks, 128 accumulators; 4 fragment reads, 4 half-fragment
// reads and 8 MFMAs per K16 step; 8 loads a stage a wave: waves 0-3 G, waves 4-7 W). Measured on
// MI355X: as fast as, or up to 6% faster than, the same schedule on W^T (the bits are the same),
// which also needed the transpose (0.13 ms at dim 1024, 0.34 at 2560).

__global__ __launch_bounds__(512) void grad_h_gemm_kernel(const uint16_t* __restrict__ G, const uint16_t* __restrict__ W,
                                                          float* __restrict__ partials, int rows, int dim, int64_t K,
                                                          int tiles, int splits, int iters_per_split) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int pairs = tiles * splits;
  const int p8 = (pairs + 7) / 8;
  const int p = (blockIdx.x % 8) * p8 + blockIdx.x / 8;
  if (p >= pairs) return;
  const int s = p / tiles, tile = p - s * tiles;
  const int tiles_n = dim / kLgTile;
  const int m0 = (tile / tiles_n) * kLgTile, n0 = (tile % tiles_n) * kLgTile;
  const int total = static_cast<int>(K / kSliceK);
  const int it0 = s * iters_per_split;
  const int n_it = max(0, min(iters_per_split, total - it0));
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int64_t k0 = static_cast<int64_t>(it0) * kSliceK;

  // Loads, 8 a wave a stage. Waves 0-3: G rows (m) 64 (w % 4) + 8 j + lane / 8 of the tile, the
  // lane's chunk (lane % 8) ^ ((row >> 1) & 7), into LDS rows 8 (8 w + j) .. of the A half (32 KB).
  // Waves 4-7: W rows (k) 16 (w % 4) + 2 j + lane / 32 of the slice, columns n0 + 8 c with
  // c = (lane % 32) ^ (4 (row & 3)), into the B half (512-byte rows), slot lane % 32.
  const uint16_t* src[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (wave < 4) {
      const int r = (wave % 4) * 64 + 8 * j + lane / 8;
      const int c = (lane % 8) ^ ((r >> 1) & 7);
      src[j] = G + static_cast<int64_t>(min(m0 + r, rows - 1)) * K + k0 + c * 8;
    } else {
      const int kr = (wave % 4) * 16 + 2 * j + lane / 32;
      const int c = (lane % 32) ^ (4 * (kr & 3));
      src[j] = W + (k0 + kr) * dim + n0 + 8 * c;
    }
  }
  const int64_t step = wave < 4 ? kSliceK : static_cast<int64_t>(kSliceK) * dim;  // elements per stage
  auto load = [&](int it, int stage, int j) {
    __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)(src[j] + it * step),
                                     (void __attribute__((address_space(3)))*)(smem + stage * kLgStage + (wave * 8 + j) * 1024),
                                     16, 0, 0);
  };
  // A fragments (m blocks) as nt_mainloop: row R0 + lane % 32, chunk 2 kk + lane / 32
  const int tx = (lane >> 5) ^ ((lane >> 1) & 7);
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem));
  const uint32_t la = lds0 + (lane & 31) * 128;
  uint32_t vk[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) vk[kk] = la + (((2 * kk) ^ tx) * 16) + wm * 128 * 128;
  // B half-fragments (n blocks) as grad_W's H operand
  const int s16 = lane & 15, s4 = s16 >> 2;
  const int lcf = ((lane >> 4) & 1) * 2 + ((s16 & 3) >> 1);
  const uint32_t rowb = (8 * (lane >> 5) + s4) * 512 + (s16 & 1) * 8;
  uint32_t bd[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) bd[b] = lds0 + kLgTile * 128 + rowb + (4 * ((2 * wn + b) ^ s4) + lcf) * 16;
#define TM_RD(dst, base, imm) asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(dst) : "v"(base), "i"(imm))
#define TM_TR(dst, base, imm) asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(dst) : "v"(base), "i"(imm))
#define TM_WAIT(a, b)                                                                                 \
  asm volatile("s_waitcnt lgkmcnt(0)"                                                                \
               : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]))
  // per K16 step: A blocks 0-3 (bf16x8); B half-fragments h = 2 b + r (bf16x4), b the n block,
  // r rows +0 / +4
  bf16x8 a0[4], a1[4];
  bf16x4 b0[4], b1[4];
  // g 0..3: A block g; 4..7: B half-fragment g - 4
  auto rd = [&](bf16x8* fa, bf16x4* fb, uint32_t so, int kk, int g) {
    if (g < 4) TM_RD(fa[g], vk[kk] + so, g * 32 * 128);
    else {
      const int h = g - 4, b = h >> 1, r = h & 1;
      TM_TR(fb[h], bd[b] + so, kk * 16 * 512 + r * 4 * 512);
    }
  };
  f32x16 acc[2][4];  // [n block][m block]
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};
  if (n_it > 0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) load(0, 0, j);
    if (n_it > 1) {
#pragma unroll
      for (int j = 0; j < 8; ++j) load(1, 1, j);
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(8));
    } else {
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    }
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int g = 0; g < 8; ++g) rd(a0, b0, 0, 0, g);
    TM_WAIT(a0, b0);
    __builtin_amdgcn_sched_barrier(0);
    auto stage = [&](int i, auto step_f) {
      constexpr bool kNext = decltype(step_f)::kNextV, kNext2 = decltype(step_f)::kNext2V;
      const int st = i & 1;
      const uint32_t soff = st * kLgStage, noff = (st ^ 1) * kLgStage;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        bf16x8* ca = (kk & 1) ? a1 : a0;
        bf16x8* na = (kk & 1) ? a0 : a1;
        bf16x4* cb = (kk & 1) ? b1 : b0;
        bf16x4* nb = (kk & 1) ? b0 : b1;
        if (kk == 3 && kNext) {
          __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
          __builtin_amdgcn_s_barrier();
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          if (kk < 3) rd(na, nb, soff, kk + 1, g);
          else if (kNext) rd(na, nb, noff, 0, g);
          if (kk == 3 && kNext2) load(i + 2, st, g);
          const int jj = g / 2, ii = g % 2;
          const bf16x8 bf = __builtin_shufflevector(cb[2 * ii], cb[2 * ii + 1], 0, 1, 2, 3, 4, 5, 6, 7);
          acc[ii][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf, ca[jj], acc[ii][jj], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
        if (kk < 3 || kNext) {
          TM_WAIT(na, nb);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    };
    int i = 0;
    for (; i + 2 < n_it; ++i) stage(i, LgFlags<true, true>{});
    if (i + 1 < n_it) stage(i++, LgFlags<true, false>{});
    if (i < n_it) stage(i, LgFlags<false, false>{});
  }
#undef TM_RD
#undef TM_TR
#undef TM_WAIT
  float* P = partials + static_cast<int64_t>(s) * rows * dim;
#pragma unroll
  for (int ii = 0; ii < 2; ++ii)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = m0 + wm * 128 + jj * 32 + (lane & 31);
        const int n = n0 + wn * 64 + ii * 32 + 8 * q + 4 * (lane >> 5);
        const f32x4 v = {acc[ii][jj][4 * q], acc[ii][jj][4 * q + 1], acc[ii][jj][4 * q + 2], acc[ii][jj][4 * q + 3]};
        *(f32x4*)(P + static_cast<int64_t>(m) * dim + n) = v;
      }
}

// ------------------------------------------------------- grad_W = grad_logits^T @ hidden
//
// fused_linear_ce.py:57 `gw = grad_logits.t() @ h` per chunk: C (vocab x dim) = G^T H with
// G = grad_logits (rows x vocab) and H = hidden (rows x dim), both stored with the contraction
// (rows) outermost. Same 256 x 256 tiles, 4 waves of 128 x 128, two 64 KB stages and the same
// schedule as logits_gemm_kernel; a stage holds 64 rows x 256 columns of each operand, 512-byte
// LDS rows whose 16-byte chunks sit at slot c ^ (4 (row & 3)). MFMA operands need 8 consecutive
// rows of one column per lane: gfx950's transposing LDS read ds_read_b64_tr_b16 gives, in each
// 16-lane group, lane i element i % 4 of the 8-byte pieces addressed by lanes i/4, i/4 + 4,
// i/4 + 8 and i/4 + 12, so with lane s addressing row s/4 at column 4 (s % 4) lane i receives
// rows 0-3 of column i; two such reads (rows +0 and +4) make a fragment. The slot swizzle puts
// the 4 rows of a read, and the 32 columns two 16-lane groups read together, on 16 different
// 16-byte bank groups. Columns past vocab or dim load a clamped (valid) column and are not stored.

constexpr int kGwOp = 64 * 512;       // one operand's stage: 64 rows x 256 bf16
constexpr int kGwStage = 2 * kGwOp;   // 64 KB

__global__ __launch_bounds__(256) void grad_w_gemm_kernel(const uint16_t* __restrict__ G, const uint16_t* __restrict__ H,
                                                          uint16_t* __restrict__ C, int V, int D, int K, int tiles_v,
                                                          int tiles_d, int gm, int gn) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int T = tiles_v * tiles_d;
  const int t8 = (T + 7) / 8;
  const int p = (blockIdx.x % 8) * t8 + blockIdx.x / 8;
  if (p >= T) return;
  int tv, td;
  lg_tile_of(p, tiles_v, tiles_d, gm, gn, tv, td);
  const int v0 = tv * kLgTile, d0 = td * kLgTile;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;  // vocab half, dim half
  const int n_it = K / kSliceK;

  // Load j of this wave, q = 16 wave + j: operand q / 32 (G, then H), rows 2 (q % 32) and
  // 2 (q % 32) + 1 of the stage; slot lane % 32 of row 2 (q % 32) + lane / 32 takes logical chunk
  // (lane % 32) ^ (4 (row & 3)).
  const uint16_t* src[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int q = wave * 16 + j;
    const int kr = 2 * (q % 32) + lane / 32;
    const int c = (lane % 32) ^ (4 * (kr & 3));
    src[j] = q < 32 ? G + static_cast<int64_t>(kr) * V + min(v0 + 8 * c, V - 8)
                    : H + static_cast<int64_t>(kr) * D + min(d0 + 8 * c, D - 8);
  }
  const int64_t step_g = static_cast<int64_t>(kSliceK) * V, step_h = static_cast<int64_t>(kSliceK) * D;
  auto load = [&](int it, int stage, int j) {
    const int q = wave * 16 + j;
    __builtin_amdgcn_global_load_lds(
        (const void __attribute__((address_space(1)))*)(src[j] + it * (q < 32 ? step_g : step_h)),
        (void __attribute__((address_space(3)))*)(smem + stage * kGwStage + q * 1024), 16, 0, 0);
  };
  // Fragment of 32-column block b at K16 step kk: lane l (s = l % 16) reads row
  // 16 kk + 8 (l / 32) + s / 4 (+4 for the second half) at column 32 b + 16 ((l / 16) % 2) + 4 (s % 4),
  // whose physical chunk is 4 (b ^ (s / 4)) + ((l / 16) % 2) * 2 + (s % 4) / 2 past the wave's 16.
  const int s16 = lane & 15, s4 = s16 >> 2;
  const int lc = ((lane >> 4) & 1) * 2 + ((s16 & 3) >> 1);
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem));
  const uint32_t rowb = (8 * (lane >> 5) + s4) * 512 + (s16 & 1) * 8;
  uint32_t bv[4], bd[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    bv[b] = lds0 + rowb + (16 * wm + 4 * (b ^ s4) + lc) * 16;
    bd[b] = lds0 + kGwOp + rowb + (16 * wn + 4 * (b ^ s4) + lc) * 16;
  }

  f32x16 acc[4][4];  // [dim block][vocab block]
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

#define TM_TR(dst, base, imm) asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(dst) : "v"(base), "i"(imm))
#define TM_WAIT16(f)                                                                                        \
  asm volatile("s_waitcnt lgkmcnt(0)"                                                                     \
               : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]), "+v"(f[6]), "+v"(f[7]), \
                 "+v"(f[8]), "+v"(f[9]), "+v"(f[10]), "+v"(f[11]), "+v"(f[12]), "+v"(f[13]), "+v"(f[14]),      \
                 "+v"(f[15]))
  // half-fragment h = 2 g + r: g < 4 -> dim block g, g >= 4 -> vocab block g - 4; r: rows +0 / +4
  bf16x4 f0[16], f1[16];
  auto rd = [&](bf16x4* f, uint32_t soff, int kk, int h) {
    const int g = h >> 1, r = h & 1;
    TM_TR(f[h], (g < 4 ? bd[g] : bv[g - 4]) + soff, kk * 16 * 512 + r * 4 * 512);
  };
#pragma unroll
  for (int j = 0; j < 16; ++j) load(0, 0, j);
  if (n_it > 1) {
#pragma unroll
    for (int j = 0; j < 16; ++j) load(1, 1, j);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(16));
  } else {
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  }
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int h = 0; h < 16; ++h) rd(f0, 0, 0, h);
  TM_WAIT16(f0);
  __builtin_amdgcn_sched_barrier(0);

  auto stage = [&](int i, auto step) {
    constexpr bool kNext = decltype(step)::kNextV, kNext2 = decltype(step)::kNext2V;
    const int s = i & 1;
    const uint32_t soff = s * kGwStage, noff = (s ^ 1) * kGwStage;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      bf16x4* cur = (kk & 1) ? f1 : f0;
      bf16x4* nxt = (kk & 1) ? f0 : f1;
      if (kk == 3 && kNext) {
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int q = 0; q < 16; ++q) {  // one half-fragment read, at most one load, one MFMA
        if (kk < 3) rd(nxt, soff, kk + 1, q);
        else if (kNext) rd(nxt, noff, 0, q);
        if (kk == 3 && kNext2) load(i + 2, s, q);
        const int ii = q / 4, jj = q % 4;
        const bf16x8 a = __builtin_shufflevector(cur[2 * ii], cur[2 * ii + 1], 0, 1, 2, 3, 4, 5, 6, 7);
        const bf16x8 b = __builtin_shufflevector(cur[8 + 2 * jj], cur[9 + 2 * jj], 0, 1, 2, 3, 4, 5, 6, 7);
        acc[ii][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[ii][jj], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (kk < 3 || kNext) {
        TM_WAIT16(nxt);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  int i = 0;
  for (; i + 2 < n_it; ++i) stage(i, LgFlags<true, true>{});
  if (i + 1 < n_it) stage(i++, LgFlags<true, false>{});
  if (i < n_it) stage(i, LgFlags<false, false>{});
#undef TM_TR
#undef TM_WAIT16

  // D[d][v] of a block: lane holds 4 consecutive dim columns of one vocab row (as the logits)
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_s_barrier();
  uint8_t* tile = smem + wave * 128 * kLgPitch;
#pragma unroll
  for (int ii = 0; ii < 4; ++ii)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int vr = jj * 32 + (lane & 31), dc = ii * 32 + 8 * q + 4 * (lane >> 5);
        u32x2 o;
        o.x = pack_bf16x2(acc[ii][jj][4 * q], acc[ii][jj][4 * q + 1]);
        o.y = pack_bf16x2(acc[ii][jj][4 * q + 2], acc[ii][jj][4 * q + 3]);
        *(u32x2*)(tile + vr * kLgPitch + dc * 2) = o;
      }
  __builtin_amdgcn_s_waitcnt(0);
  const int vb = v0 + wm * 128, db = d0 + wn * 128;
#pragma unroll 4
  for (int it = 0; it < 32; ++it) {
    const int vr = it * 4 + (lane >> 4), ch = lane & 15;
    const int v = vb + vr, d = db + ch * 8;
    if (v >= V || d >= D) continue;  // D is a multiple of 8: a group is whole or out
    const u32x4 val = *(const u32x4*)(tile + vr * kLgPitch + ch * 16);
    __builtin_nontemporal_store(val, reinterpret_cast<u32x4*>(C + static_cast<int64_t>(v) * D + d));
  }
}

// ------------------------------------------------ grad_W, persistent: one workgroup per CU
//
// grad_w_gemm_kernel's tiles, loads, transposing fragment reads and summation order (bit-identical
// results) in logits_ring_kernel's persistent form: workgroup c of XCD x runs the XCD's tile
// positions c, c + W, ...; the next tile's first two stages load during the current tile's last
// two; 8 waves, two a SIMD, wave (wm, wn) = (w / 4, w % 4) computing vocab rows wm * 128 .. +127
// and dim columns wn * 64 .. +63 (4 vocab x 2 dim blocks; 12 transposing half-fragment reads and
// 8 MFMAs per K16 step; measured on MI355X: 4-10% faster than one wave a SIMD, the same bits);
// the finished tile's accumulators are converted and staged block by block during the next tile's
// first K16 step (32 vocab rows x the wave's 64 dim columns at a time through the wave's 4 KB past
// the stages) and written as 128-byte row pieces of grad_W. For rows (K) a multiple of 128 and at
// least 256, vocab and dim multiples of 8, operands under 4 GiB; grad_w_gemm_kernel otherwise.

__global__ __launch_bounds__(512) void grad_w_ring_kernel(const uint16_t* __restrict__ G, const uint16_t* __restrict__ H,
                                                          uint16_t* __restrict__ C, int V, int D, int K, int tiles_v,
                                                          int tiles_d, int gm, int gn, int wpx) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int T = tiles_v * tiles_d;
  const int t8 = (T + 7) / 8;
  const int x = blockIdx.x % 8;
  const int pend = min((x + 1) * t8, T);
  int p = x * t8 + static_cast<int>(blockIdx.x / 8);
  if (p >= pend) return;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 2, wn = wave & 3;  // vocab half, dim quarter
  const int n_it = K / kSliceK;             // even, >= 4

  // Waves 0-3 load G (rows 16 (wave % 4) .. +15 of a stage), waves 4-7 H. Load j: stage rows
  // 16 (wave % 4) + 2 j + lane / 32, slot lane % 32 taking chunk (lane % 32) ^ (4 (row & 3)) =
  // (lane % 32) ^ (4 (lane / 32)) ^ (8 (j % 2)).
  const char* opnd = reinterpret_cast<const char*>(wave < 4 ? G : H);
  const int ld = wave < 4 ? V : D;
  const int lim8 = ld - 8;
  const uint32_t step = static_cast<uint32_t>(kSliceK) * static_cast<uint32_t>(ld) * 2u;  // bytes per stage
  uint32_t soff[8];
  int lkr = lane >> 5;
  int lc = (lane & 31) ^ (4 * (lane >> 5));
  auto set_src = [&](int v0, int d0) {
    asm volatile("" : "+v"(lkr), "+v"(lc));
    const int col0 = wave < 4 ? v0 : d0;
    const int r0 = (wave % 4) * 16;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int kr = r0 + 2 * j + lkr;
      const int c = lc ^ (8 * (j & 1));
      soff[j] = (static_cast<uint32_t>(kr) * static_cast<uint32_t>(ld) + static_cast<uint32_t>(min(col0 + 8 * c, lim8))) * 2u;
    }
  };
  auto load = [&](int it, int stage, int j) {
    __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)(opnd + (soff[j] + static_cast<uint32_t>(it) * step)),
                                     (void __attribute__((address_space(3)))*)(smem + stage * kGwStage + (wave * 8 + j) * 1024),
                                     16, 0, 0);
  };
  // transposing fragment reads as in grad_w_gemm_kernel, for the wave's 4 vocab and 2 dim blocks
  const int s16 = lane & 15, s4 = s16 >> 2;
  const int lcf = ((lane >> 4) & 1) * 2 + ((s16 & 3) >> 1);
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem));
  const uint32_t rowb = (8 * (lane >> 5) + s4) * 512 + (s16 & 1) * 8;
  uint32_t bv[4], bd[2];
#pragma unroll
  for (int b = 0; b < 4; ++b) bv[b] = lds0 + rowb + (16 * wm + 4 * (b ^ s4) + lcf) * 16;
#pragma unroll
  for (int b = 0; b < 2; ++b) bd[b] = lds0 + kGwOp + rowb + (4 * ((2 * wn + b) ^ s4) + lcf) * 16;

  // Output staging, this wave's 4 KB: vocab row r (of a vocab block's 32) at 128 r, chunk c at
  // slot c ^ ((r >> 1) & 7); read back as chunk lane % 8 of row 8 it + lane / 8.
  const uint32_t ebo = lds0 + 2 * kGwStage + wave * 4096;
  const int wr = lane & 31;
  uint32_t wa = ebo + wr * 128 + (lane >> 5) * 8;
  const uint32_t wsw = static_cast<uint32_t>((wr >> 1) & 7);
  uint32_t ra[4];
#pragma unroll
  for (int kq = 0; kq < 4; ++kq) {
    const int r = kq * 8 + (lane >> 3);
    ra[kq] = ebo + r * 128 + (((lane & 7) ^ ((r >> 1) & 7)) << 4);
  }
  uint32_t sl = static_cast<uint32_t>(((lane >> 3) * D + (lane & 7) * 8) * 2);

#define TM_TR(dst, base, imm) asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(dst) : "v"(base), "i"(imm))
#define TM_WAIT12(f)                                                                                        \
  asm volatile("s_waitcnt lgkmcnt(0)"                                                                     \
               : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]), "+v"(f[6]), "+v"(f[7]), \
                 "+v"(f[8]), "+v"(f[9]), "+v"(f[10]), "+v"(f[11]))
  // half-fragment h = 2 g + r: g < 2 -> dim block g, g >= 2 -> vocab block g - 2; r: rows +0 / +4
  bf16x4 f0[12], f1[12];
  auto rd = [&](bf16x4* f, uint32_t so, int kk, int h) {
    const int g = h >> 1, r = h & 1;
    TM_TR(f[h], (g < 2 ? bd[g] : bv[g - 2]) + so, kk * 16 * 512 + r * 4 * 512);
  };
  f32x16 acc[2][4];  // [dim block][vocab block]
  int pv0 = 0, pd0 = 0;  // origin of the tile whose output is being written

  // block (ii, jj) -> staging (and the next tile's first MFMA on it), as in logits_ring_kernel

  auto epi_block = [&](int ii, int jj, bool mfma, bf16x4* cur) {
    asm volatile("" : "+v"(acc[ii][jj]));
    u32x2 o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      o[q].x = pack_bf16x2(acc[ii][jj][4 * q], acc[ii][jj][4 * q + 1]);
      o[q].y = pack_bf16x2(acc[ii][jj][4 * q + 2], acc[ii][jj][4 * q + 3]);
    }
    if (mfma) {
      asm volatile("" : "+v"(cur[2 * ii]) : "v"(o[0]), "v"(o[1]), "v"(o[2]), "v"(o[3]));
      const bf16x8 a = __builtin_shufflevector(cur[2 * ii], cur[2 * ii + 1], 0, 1, 2, 3, 4, 5, 6, 7);
      const bf16x8 b = __builtin_shufflevector(cur[4 + 2 * jj], cur[5 + 2 * jj], 0, 1, 2, 3, 4, 5, 6, 7);
      acc[ii][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, f32x16{}, 0, 0, 0);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t a = wa + (((static_cast<uint32_t>(ii * 4 + q)) ^ wsw) << 4);
      asm volatile("ds_write_b64 %0, %1" ::"v"(a), "v"(o[q]) : "memory");
    }
  };
  // vocab block jj (32 rows x the wave's 64 dim columns) -> grad_W, 16 bytes a lane (D % 8 == 0)
  auto epi_store = [&](int jj) {
    u32x4 v[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) asm volatile("ds_read_b128 %0, %1" : "=v"(v[it]) : "v"(ra[it]));
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]));
    const int rows_left = V - (pv0 + wm * 128 + jj * 32), cols_left = D - (pd0 + wn * 64);
    char* qb = reinterpret_cast<char*>(C) + (static_cast<int64_t>(pv0 + wm * 128 + jj * 32) * D + pd0 + wn * 64) * 2;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      if (it * 8 + (lane >> 3) < rows_left && (lane & 7) * 8 < cols_left)
        __builtin_nontemporal_store(v[it], reinterpret_cast<u32x4*>(qb + (sl + static_cast<uint32_t>(it * 8 * D * 2))));
    }
  };

  int tv, td;
  lg_tile_of(p, tiles_v, tiles_d, gm, gn, tv, td);
  int v0 = tv * kLgTile, d0 = td * kLgTile;
  set_src(v0, d0);
#pragma unroll
  for (int j = 0; j < 8; ++j) load(0, 0, j);
#pragma unroll
  for (int j = 0; j < 8; ++j) load(1, 1, j);
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(8));
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int h = 0; h < 12; ++h) rd(f0, 0, 0, h);
  TM_WAIT12(f0);
  __builtin_amdgcn_sched_barrier(0);

  int pn = p, v0n = v0, d0n = d0;
  bool has_next = false;
  // one tile, as in logits_ring_kernel
  auto tile = [&](auto epi_first) {
    constexpr bool kEpiFirst = decltype(epi_first)::value;
    asm volatile("" : "+v"(wa), "+v"(ra[0]), "+v"(ra[1]), "+v"(ra[2]), "+v"(ra[3]), "+v"(sl));
    pn = p + wpx;
    has_next = pn < pend;
    int tvn, tdn;
    lg_tile_of(has_next ? pn : p, tiles_v, tiles_d, gm, gn, tvn, tdn);
    v0n = tvn * kLgTile;
    d0n = tdn * kLgTile;

    auto stage = [&](int i, auto step) {
      constexpr bool kNext2 = decltype(step)::kNext2V, kPre = decltype(step)::kPreV;
      constexpr bool kFirst = decltype(step)::kFirstV, kEpi = decltype(step)::kEpiV;
      const int s = i & 1;
      const uint32_t so = s * kGwStage, noff = (s ^ 1) * kGwStage;
      if (kPre) {
        set_src(v0n, d0n);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        bf16x4* cur = (kk & 1) ? f1 : f0;
        bf16x4* nxt = (kk & 1) ? f0 : f1;
        if (kEpi && kk == 0) {
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
            for (int ii = 0; ii < 2; ++ii) {
              const int bi = jj * 2 + ii;
              rd(nxt, so, 1, bi);
              if (bi < 4) rd(nxt, so, 1, 8 + bi);
              epi_block(ii, jj, true, cur);
              __builtin_amdgcn_sched_barrier(0);
            }
            epi_store(jj);
            __builtin_amdgcn_sched_barrier(0);
          }
          TM_WAIT12(nxt);
          __builtin_amdgcn_sched_barrier(0);
          continue;
        }
        if (kk == 3) {
          __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
          __builtin_amdgcn_s_barrier();
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {  // one MFMA, one or two half-fragment reads, at most one load
          if (kk < 3) {
            rd(nxt, so, kk + 1, q);
            if (q < 4) rd(nxt, so, kk + 1, 8 + q);
          } else {
            rd(nxt, noff, 0, q);
            if (q < 4) rd(nxt, noff, 0, 8 + q);
          }
          if (kk == 3 && kNext2) {
            const int it2 = i + 2 >= n_it ? i + 2 - n_it : i + 2;
            load(it2, s, q);
          }
          const int jj = q / 2, ii = q % 2;
          const bf16x8 a = __builtin_shufflevector(cur[2 * ii], cur[2 * ii + 1], 0, 1, 2, 3, 4, 5, 6, 7);
          const bf16x8 b = __builtin_shufflevector(cur[4 + 2 * jj], cur[5 + 2 * jj], 0, 1, 2, 3, 4, 5, 6, 7);
          if (kFirst && kk == 0)
            acc[ii][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, f32x16{}, 0, 0, 0);
          else
            acc[ii][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[ii][jj], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
        TM_WAIT12(nxt);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    stage(0, RgFlags<true, false, true, kEpiFirst>{});
    for (int i = 1; i < n_it - 2; ++i) stage(i, RgFlags<true, false, false, false>{});
    stage(n_it - 2, RgFlags<true, true, false, false>{});
    stage(n_it - 1, RgFlags<true, false, false, false>{});
    pv0 = v0;
    pd0 = d0;
  };
  tile(RgBool<false>{});
  while (has_next) {
    p = pn;
    v0 = v0n;
    d0 = d0n;
    __builtin_amdgcn_sched_barrier(0);
    tile(RgBool<true>{});
  }
  // the last tile's output; then the redundant reload of that tile's first stages completes
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) epi_block(ii, jj, false, f0);
    epi_store(jj);
  }
  __builtin_amdgcn_s_waitcnt(0);
#undef TM_TR
#undef TM_WAIT12
}


bool grad_w_ring_fits(int64_t rows, int64_t vocab, int64_t dim) {
  return rows % 128 == 0 && rows >= 256 && vocab % 8 == 0 && dim % 8 == 0 && rows * vocab * 2 < (int64_t(1) << 32) &&
         rows * dim * 2 < (int64_t(1) << 32) && 32 * dim * 2 < (int64_t(1) << 32);
}

// Tile groups per XCD round (gm row tiles x gn weight panels, gm gn = 32), chosen from a sweep of
// the logits ring kernel on MI355X (V = 151,936; TFLOP/s of the best against the next best):
//   dim <= 1024: 1 x 32 up to 4 row tiles (1063 against 855 for 4 x 8 at 1024 rows: the hidden
//                chunk sits in every XCD's L2 and a round takes one row of 32 panels), 2 x 16 up
//                to 8, 4 x 8 above;
//   dim <= 2560: 2 x 16 up to 8 row tiles (1048 against 899 for 1 x 32 at 1024 x 2560), 4 x 8
//                above;
//   dim <= 4096: 4 x 8 (1118 against 1008 for 1 x 32 at 1024 x 4096);
//   wider:       8 x 4 from 8 row tiles (1195 against 1125 for 4 x 8 at 8192 x 5120), 4 x 8 below.
// Wider panels (256 x dim) leave fewer in an XCD's 4 MB L2, so rounds share each panel among more
// tiles.
void logits_groups(int64_t tiles_m, int64_t dim, int& gm, int& gn) {
  if (dim <= 1024) gm = tiles_m <= 4 ? 1 : (tiles_m <= 8 ? 2 : 4);
  else if (dim <= 2560) gm = tiles_m <= 8 ? 2 : 4;
  else if (dim <= 4096) gm = 4;
  else gm = tiles_m >= 8 ? 8 : 4;
  gn = 32 / gm;
}

// Splits of the K range, chosen by a cost model of the launch. One workgroup (128 KB of LDS) fits
// a CU, so tiles x S workgroups run in ceil(tiles x S / 256) rounds; a workgroup takes about
// 1.7 us per 64-deep K slice (256 x 256 x 64 MFMA work at the main loop's pace) plus about 8 us
// to store its 256 KB partial tile, and the reduction reads S x rows x dim fp32 partials at about
// 5 TB/s. For the Qwen3-0.6B head (dim 1024) the model picks S = 16 for a 1024-row chunk
// (16 tiles, 256 workgroups), 4 for 4096 rows and 2 for 8192 rows (128 tiles).
int64_t splits_for(int64_t rows, int64_t vocab, int64_t dim) {
  const int64_t tiles = (rows / kTile) * (dim / kTile);
  const int64_t iters = vocab / kSliceK;
  int64_t best = 1;
  double best_us = 0.0;
  for (int64_t s = 1; s <= 256; ++s) {
    const int64_t rounds = (tiles * s + 255) / 256;
    const double us = static_cast<double>(rounds) * (1.7 * static_cast<double>((iters + s - 1) / s) + 8.0) +
                      static_cast<double>(s) * static_cast<double>(rows * dim) * 4.0 / 5e6;
    if (s == 1 || us < best_us) {
      best = s;
      best_us = us;
    }
  }
  return best;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The GEMM kernels' dynamic LDS (128-160 KB) exceeds the 64 KB default:
// the attribute is set once per device and kernel, with that device current, before the first
// launch there. The device's CU count (for the ring kernels' workgroups per XCD) is read then.
constexpr int kMaxDevices = 64;
std::mutex g_lds_mu;
bool g_lds_set[5][kMaxDevices] = {};
int g_cus[kMaxDevices] = {};

// which: 0 grad_h_gemm_kernel, 1 logits_gemm_kernel, 2 grad_w_gemm_kernel, 3 logits_ring_kernel,
// 4 grad_w_ring_kernel.
// `cus`, when given, receives the device's CU count.
hipError_t allow_lds(hipStream_t stream, int which, int* cus = nullptr) {
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_lds_mu);
  if (g_lds_set[which][dev]) {
    if (cus) *cus = g_cus[dev];
    return hipSuccess;
  }
  int cur = -1;
  e = hipGetDevice(&cur);
  if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
  const void* fn[5] = {reinterpret_cast<const void*>(grad_h_gemm_kernel), reinterpret_cast<const void*>(logits_gemm_kernel),
                       reinterpret_cast<const void*>(grad_w_gemm_kernel), reinterpret_cast<const void*>(logits_ring_kernel),
                       reinterpret_cast<const void*>(grad_w_ring_kernel)};
  const int bytes[5] = {2 * kLgStage, kLgLds, kLgLds, kRgLds, kRgLds};
  if (e == hipSuccess) e = hipFuncSetAttribute(fn[which], hipFuncAttributeMaxDynamicSharedMemorySize, bytes[which]);
  if (e == hipSuccess && g_cus[dev] == 0) e = hipDeviceGetAttribute(&g_cus[dev], hipDeviceAttributeMultiprocessorCount, dev);
  if (cur >= 0 && cur != dev) {
    const hipError_t back = hipSetDevice(cur);
    if (e == hipSuccess) e = back;
  }
  if (e == hipSuccess) {
    g_lds_set[which][dev] = true;
    if (cus) *cus = g_cus[dev];
  }
  return e;
}

}  // namespace

extern "C" {

size_t tm_ce_grad_h_workspace_bytes(int64_t rows, int64_t vocab, int64_t dim) {
  if (rows <= 0 || dim <= 0 || vocab <= 0 || rows % kTile || dim % kTile || vocab % kSliceK) return 0;
  return static_cast<size_t>(splits_for(rows, vocab, dim)) * rows * dim * sizeof(float);
}

int tm_ce_grad_h_bf16(uint16_t* d_grad_h, const uint16_t* d_grad_logits, const uint16_t* d_w, int64_t rows,
                      int64_t vocab, int64_t dim, void* d_ws, size_t ws_bytes, void* stream) {
  if (rows <= 0 || dim <= 0 || vocab <= 0 || rows % kTile || dim % kTile || vocab % kSliceK)
    return gemm_fail(TM_EINVAL,
                     "tm_ce_grad_h_bf16: rows %lld and dim %lld must be positive multiples of %d, vocab %lld "
                     "of %d", (long long)rows, (long long)dim, kTile, (long long)vocab, kSliceK);
  if (rows > (1 << 20) || dim > (1 << 16))
    return gemm_fail(TM_EINVAL, "tm_ce_grad_h_bf16: rows %lld or dim %lld too large", (long long)rows,
                     (long long)dim);
  if (!d_grad_h || !d_grad_logits || !d_w || !d_ws)
    return gemm_fail(TM_EINVAL, "tm_ce_grad_h_bf16: null pointer");
  if (!aligned16(d_grad_h) || !aligned16(d_grad_logits) || !aligned16(d_w) || !aligned16(d_ws))
    return gemm_fail(TM_EINVAL, "tm_ce_grad_h_bf16: pointers must be 16-byte aligned");
  if (ws_bytes < tm_ce_grad_h_workspace_bytes(rows, vocab, dim))
    return gemm_fail(TM_EINVAL, "tm_ce_grad_h_bf16: workspace of %zu bytes, %zu needed", ws_bytes,
                     tm_ce_grad_h_workspace_bytes(rows, vocab, dim));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t splits = splits_for(rows, vocab, dim);
  const int64_t tiles = (rows / kTile) * (dim / kTile);
  const int64_t total_iters = vocab / kSliceK;
  const int64_t per = (total_iters + splits - 1) / splits;
  const hipError_t lds = allow_lds(s, 0);
  if (lds != hipSuccess)
    return gemm_fail(TM_ELAUNCH, "tm_ce_grad_h_bf16: LDS attribute: %s", hipGetErrorString(lds));
  float* partials = static_cast<float*>(d_ws);
  hipLaunchKernelGGL(grad_h_gemm_kernel, dim3(static_cast<uint32_t>((tiles * splits + 7) / 8 * 8)), dim3(512),
                     2 * kLgStage, s, d_grad_logits, d_w, partials, static_cast<int>(rows), static_cast<int>(dim),
                     vocab, static_cast<int>(tiles), static_cast<int>(splits), static_cast<int>(per));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return gemm_fail(TM_ELAUNCH, "grad_h_gemm_kernel: launch failed: %s", hipGetErrorString(e));
  const int64_t n = rows * dim;
  hipLaunchKernelGGL(grad_h_reduce_kernel, dim3(static_cast<uint32_t>((n / 4 + 255) / 256)), dim3(256), 0, s,
                     partials, d_grad_h, n, static_cast<int>(splits));
  e = hipGetLastError();
  if (e != hipSuccess) return gemm_fail(TM_ELAUNCH, "grad_h_reduce_kernel: launch failed: %s", hipGetErrorString(e));
  return TM_OK;
}

int tm_ce_logits_bf16(uint16_t* d_logits, const uint16_t* d_hidden, const uint16_t* d_weight, int64_t rows,
                      int64_t vocab, int64_t dim, void* stream) {
  if (rows <= 0 || vocab <= 0 || dim <= 0 || dim % kSliceK)
    return gemm_fail(TM_EINVAL, "tm_ce_logits_bf16: rows %lld and vocab %lld must be positive, dim %lld a positive "
                     "multiple of %d", (long long)rows, (long long)vocab, (long long)dim, kSliceK);
  const int64_t tiles_m = (rows + kLgTile - 1) / kLgTile, tiles_n = (vocab + kLgTile - 1) / kLgTile;
  if (rows > 0x7FFFFFFF || vocab > 0x7FFFFFFF || dim > 0x7FFFFFFF || tiles_m * tiles_n > 0x7FFFFFF0)
    return gemm_fail(TM_EINVAL, "tm_ce_logits_bf16: %lld x %lld x %lld is too large", (long long)rows,
                     (long long)vocab, (long long)dim);
  if (!d_logits || !d_hidden || !d_weight) return gemm_fail(TM_EINVAL, "tm_ce_logits_bf16: null pointer");
  if (!aligned16(d_logits) || !aligned16(d_hidden) || !aligned16(d_weight))
    return gemm_fail(TM_EINVAL, "tm_ce_logits_bf16: pointers must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  int gm, gn;
  logits_groups(tiles_m, dim, gm, gn);
  if (logits_ring_fits(rows, vocab, dim)) {
    int cus = 0;
    const hipError_t lds = allow_lds(s, 3, &cus);
    if (lds != hipSuccess)
      return gemm_fail(TM_ELAUNCH, "tm_ce_logits_bf16: LDS attribute: %s", hipGetErrorString(lds));
    const int wpx = cus >= 16 ? cus / 8 : 1;  // one workgroup per CU of each XCD
    hipLaunchKernelGGL(logits_ring_kernel, dim3(static_cast<uint32_t>(8 * wpx)), dim3(512), kRgLds, s, d_hidden,
                       d_weight, d_logits, static_cast<int>(rows), static_cast<int>(vocab), static_cast<int>(dim),
                       static_cast<int>(tiles_m), static_cast<int>(tiles_n), gm, gn, wpx);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return gemm_fail(TM_ELAUNCH, "logits_ring_kernel: launch failed: %s", hipGetErrorString(e));
    return TM_OK;
  }
  const hipError_t lds = allow_lds(s, 1);
  if (lds != hipSuccess)
    return gemm_fail(TM_ELAUNCH, "tm_ce_logits_bf16: LDS attribute: %s", hipGetErrorString(lds));
  const int64_t grid = (tiles_m * tiles_n + 7) / 8 * 8;
  hipLaunchKernelGGL(logits_gemm_kernel, dim3(static_cast<uint32_t>(grid)), dim3(256), kLgLds, s, d_hidden, d_weight,
                     d_logits, static_cast<int>(rows), static_cast<int>(vocab), static_cast<int>(dim),
                     static_cast<int>(tiles_m), static_cast<int>(tiles_n), gm, gn);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return gemm_fail(TM_ELAUNCH, "logits_gemm_kernel: launch failed: %s", hipGetErrorString(e));
  return TM_OK;
}

int tm_ce_grad_w_bf16(uint16_t* d_grad_w, const uint16_t* d_grad_logits, const uint16_t* d_hidden, int64_t rows,
                      int64_t vocab, int64_t dim, void* stream) {
  if (rows <= 0 || vocab <= 0 || dim <= 0 || rows % kSliceK || vocab % 8 || dim % 8)
    return gemm_fail(TM_EINVAL, "tm_ce_grad_w_bf16: rows %lld must be a positive multiple of %d, vocab %lld and dim "
                     "%lld positive multiples of 8", (long long)rows, kSliceK, (long long)vocab, (long long)dim);
  const int64_t tiles_v = (vocab + kLgTile - 1) / kLgTile, tiles_d = (dim + kLgTile - 1) / kLgTile;
  if (rows > 0x7FFFFFFF || vocab > 0x7FFFFFFF || dim > 0x7FFFFFFF || tiles_v * tiles_d > 0x7FFFFFF0)
    return gemm_fail(TM_EINVAL, "tm_ce_grad_w_bf16: %lld x %lld x %lld is too large", (long long)rows,
                     (long long)vocab, (long long)dim);
  if (!d_grad_w || !d_grad_logits || !d_hidden) return gemm_fail(TM_EINVAL, "tm_ce_grad_w_bf16: null pointer");
  if (!aligned16(d_grad_w) || !aligned16(d_grad_logits) || !aligned16(d_hidden))
    return gemm_fail(TM_EINVAL, "tm_ce_grad_w_bf16: pointers must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int gn = static_cast<int>(tiles_d < 4 ? tiles_d : 4), gm = 32 / gn;  // a round of 32: 8 x 4
  if (grad_w_ring_fits(rows, vocab, dim)) {
    int cus = 0;
    const hipError_t lds = allow_lds(s, 4, &cus);
    if (lds != hipSuccess)
      return gemm_fail(TM_ELAUNCH, "tm_ce_grad_w_bf16: LDS attribute: %s", hipGetErrorString(lds));
    const int wpx = cus >= 16 ? cus / 8 : 1;
    hipLaunchKernelGGL(grad_w_ring_kernel, dim3(static_cast<uint32_t>(8 * wpx)), dim3(512), kRgLds, s, d_grad_logits,
                       d_hidden, d_grad_w, static_cast<int>(vocab), static_cast<int>(dim), static_cast<int>(rows),
                       static_cast<int>(tiles_v), static_cast<int>(tiles_d), gm, gn, wpx);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return gemm_fail(TM_ELAUNCH, "grad_w_ring_kernel: launch failed: %s", hipGetErrorString(e));
    return TM_OK;
  }
  const hipError_t lds = allow_lds(s, 2);
  if (lds != hipSuccess)
    return gemm_fail(TM_ELAUNCH, "tm_ce_grad_w_bf16: LDS attribute: %s", hipGetErrorString(lds));
  const int64_t grid = (tiles_v * tiles_d + 7) / 8 * 8;
  hipLaunchKernelGGL(grad_w_gemm_kernel, dim3(static_cast<uint32_t>(grid)), dim3(256), kLgLds, s, d_grad_logits,
                     d_hidden, d_grad_w, static_cast<int>(vocab), static_cast<int>(dim), static_cast<int>(rows),
                     static_cast<int>(tiles_v), static_cast<int>(tiles_d), gm, gn);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return gemm_fail(TM_ELAUNCH, "grad_w_gemm_kernel: launch failed: %s", hipGetErrorString(e));
  return TM_OK;
}

}  // extern "C"
