// tfgfa_fwd.hip - causal FlashAttention forward for MI355X (gfx950), bf16 in/out.
//
// Replaces the reference's device kernel (src/cpp/headers/v1_implementation.hpp:12-171),
// its tile constants (src/cpp/headers/common_types.hpp:18-38) and its host launcher
// (src/cpp/v1.cu:4-38).  The math is the reference's causal attention
// softmax(scale * Q K^T) V with the diagonal included (v1_implementation.hpp:105-112,
// src/py/model_inference.py:68-75), computed blockwise with an online softmax
// (v1_implementation.hpp:115-158; rescale algebra as src/py/triton_implementation.py:129-160),
// plus the per-row natural-log log-sum-exp (triton_implementation.py:153-154).
//
// Work decomposition
//   One workgroup = 4 waves = one 128-row query block of one (batch, head).  Each wave owns
//   32 query rows and walks the key/value sequence in 64-key tiles.  Tiles wholly above the
//   causal diagonal are never loaded (per workgroup) or computed (per wave); only tiles that
//   cross the diagonal or the sequence end apply an element mask.  Workgroups are issued
//   heaviest query block first.
//
// Memory pipeline
//   K and V tiles go from HBM straight into LDS (buffer_load_dwordx4 ... lds: each lane's
//   16 B land at LDS base + 16*lane), through a ring of 3 stages, so two tiles are in flight
//   while one is computed.  No registers or VALU work are spent on staging.  Loads past the
//   sequence end return zero (buffer range check), which is the zero-fill of partial tiles.
//   One barrier per tile: wait for this wave's loads of the tile, barrier (all waves' loads
//   landed, all waves done with the stage about to be refilled), issue the loads two tiles
//   ahead, compute.
//
// MFMA chaining without an LDS round trip (v_mfma_f32_32x32x16_bf16, fp32 accumulate)
//   S^T = K . Q^T  : A = K tile rows (32 keys x 16 d, ds_read_b128), B = Q^T (16 d x 32
//                    queries, held in registers).  Accumulator lane l holds query l%32 and 16
//                    of the 32 keys, so a row's max/sum is an in-lane reduction plus one
//                    v_permlane32_swap with lane l^32.
//   O^T = V^T . P^T: B = P^T comes straight from the S^T accumulator registers (the
//                    contraction order over keys is relabelled to match), A = V^T is read
//                    from the row-major V tile with ds_read_b64_tr_b16.  O^T's lane l again
//                    holds query l%32.
//   Lane layouts of 32x32x16 (K = 16 per instruction):
//     A[i][k]: lane = i + 32*(k/8), element k%8        B[k][j]: lane = j + 32*(k/8), element k%8
//     D[i][j]: lane = j + 32*((i/4)%2), register 4*(i/8) + i%4
//   ds_read_b64_tr_b16, per group of 16 lanes: lane j supplies 4 b16 values M[j][0..3]; lane i
//   receives M[4e + i/4][i%4], e = 0..3.  With source lane j pointing at
//   V[kb + j/4][D + 4*(j%4) .. +3], lane i receives V[kb + e][D + i]: 4 consecutive keys of
//   one d, the V^T operand layout.
//
// LDS layouts (per stage: K tile 8 KiB then V tile 8 KiB, 128 B per key row)
//   16-B chunk c of row r is stored at chunk c ^ swz(r).  K: swz = (r ^ (r >> 3)) & 7 makes any
//   8 (or 16) consecutive rows of one logical chunk hit distinct banks for the ds_read_b128
//   A-operand reads.  V: swz = 2*(r & 3) makes the 4-row x 32-B footprint of a transposing read
//   group (and of two groups side by side) hit distinct banks.
//
// Softmax runs in the exp2 domain: scores are scaled by scale*log2(e) inside one FMA, the
// running max m and sum l are per-lane registers, and LSE = (m + log2 l) * ln 2.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <string.h>

#include <mutex>

#include "tfgfa.h"

namespace tfgfa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kD = 64;                      // head dimension (the only compiled one)
constexpr int kWaves = 4;                   // waves per workgroup
constexpr int kThreads = kWaves * 64;       // 256
constexpr int kWaveRows = 32;               // query rows per wave (one MFMA column block)
constexpr int kBlockRows = kWaves * kWaveRows;  // 128 query rows per workgroup
constexpr int kTileKeys = 64;               // keys per K/V tile
constexpr int kKRowBytes = kD * 2;          // 128 B per K or V row
constexpr int kHalfTileBytes = kTileKeys * kKRowBytes;  // 8 KiB (K or V)
constexpr int kTileBytes = 2 * kHalfTileBytes;          // 16 KiB per stage
constexpr int kStages = 3;
constexpr int kSmemBytes = kStages * kTileBytes;        // 48 KiB
constexpr int kLoadsPerWave = 2 * (kHalfTileBytes / 1024) / kWaves;  // 1 KiB per load instr: 4

// The running max used as the exp2 offset is only moved when a row's tile max exceeds it by
// more than this (log2 units), so most tiles skip the O/l rescale; probabilities then stay
// below 2^8, well inside bf16/fp32 range.
constexpr float kRescaleThreshold = 8.0f;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Row reductions across the two lane halves (lane l and l^32 hold the same query row).
// v_permlane32_swap(x, y) exchanges the upper half of x with the lower half of y, so with
// both operands equal to x each lane ends up with its own value in one result and the
// partner's in the other: max3(x, r0, r1) is the pair's max and r0 + r1 the pair's sum.
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(x, fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])));
}

__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ int swz_k(int row) { return (row ^ (row >> 3)) & 7; }
__device__ __forceinline__ int swz_v(int row) { return (row & 3) << 1; }

// Buffer resource over one head's (N, 64) bf16 rows: loads at byte offsets >= N*128 return
// zero.  The whole offset is kept in the VGPR operand so the range check covers all of it.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t head_rsrc(const __bf16* base, int N) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<__bf16*>(base), (short)0, N * kKRowBytes,
                                           0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}

// This wave's share of one tile: K and V rows [8*(2w), 8*(2w+2)) as 1-KiB LDS blocks.  Lane i
// of a block fills physical chunk i%8 of row i/8, so it fetches the logical chunk that the
// swizzle maps there.
__device__ __forceinline__ void issue_tile(__amdgpu_buffer_rsrc_t kr, __amdgpu_buffer_rsrc_t vr,
                                           unsigned char* stage, int k0, int wave, int lane) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int blk = 2 * wave + i;
    const int row = blk * 8 + (lane >> 3);
    const int pc = lane & 7;
    const int goff = (k0 + row) * kKRowBytes;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, (lds_void*)(stage + blk * 1024), 16,
                                             goff + ((pc ^ swz_k(row)) << 4), 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(vr, (lds_void*)(stage + kHalfTileBytes + blk * 1024),
                                             16, goff + ((pc ^ swz_v(row)) << 4), 0, 0, 0);
  }
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Per-wave state carried across tiles.
struct WaveState {
  bf16x8 qop[4];   // Q^T operand: Q[qrow][16c + 8h .. +7]
  f32x16 o0, o1;   // O^T accumulators: d = 0..31 and d = 32..63
  float m_run;     // exp2 offset (running max of scale*log2e*s, moved lazily)
  float l_run;     // running sum of exp2(scale*log2e*s - m_run)
  int koff[2][4];  // K A-operand LDS offsets (within a stage)
  int voff[2][2];  // V^T transposing-read LDS offsets (within a stage, c4 = 0)
};

// One 64-key tile for one wave: S^T = K Q^T, mask (kMask), online softmax, O^T += V^T P^T.
// kStage is the LDS ring slot, so every LDS address is a per-lane base plus an immediate.
template <int kStage, bool kMask>
__device__ __forceinline__ void tile_step(WaveState& w, const unsigned char* smem, int lim,
                                          float scale_log2) {
  const unsigned char* stage = smem + kStage * kTileBytes;

  // S^T for keys k0 + [0,32) (s0) and k0 + [32,64) (s1).
  f32x16 s0, s1;
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    s0[t] = 0.f;
    s1[t] = 0.f;
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(stage + w.koff[0][c]);
    const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(stage + w.koff[1][c]);
    s0 = mfma32(a0, w.qop[c], s0);
    s1 = mfma32(a1, w.qop[c], s1);
  }

  // Register t of s0 is key k0 + 8(t/4) + 4h + t%4 (s1: +32); lim is the last visible key of
  // the lane's row relative to k0 + 4h.
  if (kMask) {
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int kk = 8 * (t >> 2) + (t & 3);
      s0[t] = kk > lim ? -INFINITY : s0[t];
      s1[t] = kk + 32 > lim ? -INFINITY : s1[t];
    }
  }

  // Row max over this lane's 32 scores, then across the lane pair.
  float mx = fmaxf(s0[0], fmaxf(s0[1], s0[2]));
#pragma unroll
  for (int t = 3; t < 15; t += 2) mx = fmaxf(mx, fmaxf(s0[t], s0[t + 1]));
  mx = fmaxf(mx, fmaxf(s0[15], s1[0]));
#pragma unroll
  for (int t = 1; t < 15; t += 2) mx = fmaxf(mx, fmaxf(s1[t], s1[t + 1]));
  mx = fmaxf(mx, s1[15]);
  mx = pair_max(mx);

  // Lazy rescale: every active tile has an unmasked key in every row (the tile starts at or
  // below the wave's first row), so the tile max is finite and the first tile always moves
  // m_run off -inf.
  const float m_tile = mx * scale_log2;
  const bool grow = m_tile > w.m_run + kRescaleThreshold;
  if (__builtin_amdgcn_ballot_w64(grow) != 0) {
    const float m_new = grow ? m_tile : w.m_run;
    const float alpha = __builtin_amdgcn_exp2f(w.m_run - m_new);
    w.m_run = m_new;
    w.l_run *= alpha;
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      w.o0[t] *= alpha;
      w.o1[t] *= alpha;
    }
  }

  // P = exp2(scale*log2e*s - m_run) in fp32; the row sum l is taken in fp32 (four partial
  // sums to shorten the dependency chain), then P is rounded to bf16 for the MFMA.
  // Chunk c4 covers keys 16*c4 .. 16*c4+15 of the tile; this lane's 8 values are
  // accumulator registers 8*(c4&1) .. +7 of s0 (c4 < 2) or s1.
  const float neg_m = -w.m_run;
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    s0[t] = __builtin_amdgcn_exp2f(fmaf(s0[t], scale_log2, neg_m));
    s1[t] = __builtin_amdgcn_exp2f(fmaf(s1[t], scale_log2, neg_m));
  }
  float ps0 = s0[0], ps1 = s0[1], ps2 = s1[0], ps3 = s1[1];
#pragma unroll
  for (int t = 2; t < 16; t += 2) {
    ps0 += s0[t];
    ps1 += s0[t + 1];
    ps2 += s1[t];
    ps3 += s1[t + 1];
  }
  w.l_run += pair_sum((ps0 + ps1) + (ps2 + ps3));
  bf16x8 pb[4];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    pb[0][e] = (__bf16)s0[e];
    pb[1][e] = (__bf16)s0[8 + e];
    pb[2][e] = (__bf16)s1[e];
    pb[3][e] = (__bf16)s1[8 + e];
  }

  // O^T += V^T P^T.  Element e of chunk c4 in lane half h is key 16*c4 + 8*(e/4) + 4*h + e%4:
  // two transposing reads of 4 keys each.
#pragma unroll
  for (int c4 = 0; c4 < 4; ++c4) {
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)(stage + w.voff[dt][0] + c4 * 16 * kKRowBytes));
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)(stage + w.voff[dt][1] + c4 * 16 * kKRowBytes));
      const bf16x8 va =
          __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      if (dt == 0)
        w.o0 = mfma32(va, pb[c4], w.o0);
      else
        w.o1 = mfma32(va, pb[c4], w.o1);
    }
  }
}

// Pipeline step for tile j held in ring slot kStage: wait for the tile, barrier, refill the
// slot freed by tile j-1 with tile j+2, then compute (unless the wave has no visible key).
template <int kStage>
__device__ __forceinline__ void pipeline_step(WaveState& w, unsigned char* smem, int j, int nT,
                                              __amdgpu_buffer_rsrc_t k_rsrc,
                                              __amdgpu_buffer_rsrc_t v_rsrc, int wave, int lane,
                                              int q0, int N, int causal, int last_key, int h,
                                              float scale_log2) {
  if (j + 1 < nT)
    wait_vmcnt<kLoadsPerWave>();  // tile j landed; tile j+1 may still be in flight
  else
    wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();
  if (j + 2 < nT)
    issue_tile(k_rsrc, v_rsrc, smem + ((kStage + 2) % kStages) * kTileBytes, (j + 2) * kTileKeys,
               wave, lane);

  const int k0 = j * kTileKeys;
  if (q0 >= N || (causal && k0 > q0 + kWaveRows - 1)) return;  // wave-uniform
  if ((causal && k0 + kTileKeys - 1 > q0) || (k0 + kTileKeys > N))
    tile_step<kStage, true>(w, smem, last_key - k0 - 4 * h, scale_log2);
  else
    tile_step<kStage, false>(w, smem, 0, scale_log2);
}

__global__ __launch_bounds__(kThreads, 2) void fwd_kernel(
    const __bf16* __restrict__ Q, const __bf16* __restrict__ K, const __bf16* __restrict__ V,
    __bf16* __restrict__ O, float* __restrict__ LSE, int BH, int N, int nQB, float scale_log2,
    int causal) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[kSmemBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31;
  const int h = lane >> 5;

  // Heaviest (last) query blocks first: with causal masking block qb needs qb+1 key blocks.
  const int bid = blockIdx.x;
  const int qb = nQB - 1 - bid / BH;
  const int bh = bid % BH;

  const size_t head_off = (size_t)bh * N * kD;
  const __amdgpu_buffer_rsrc_t q_rsrc = head_rsrc(Q + head_off, N);
  const __amdgpu_buffer_rsrc_t k_rsrc = head_rsrc(K + head_off, N);
  const __amdgpu_buffer_rsrc_t v_rsrc = head_rsrc(V + head_off, N);

  const int q0 = qb * kBlockRows + wave * kWaveRows;  // first query row of this wave
  const int qrow = q0 + r32;                          // this lane's query row

  const int kv_end = causal ? min(N, (qb + 1) * kBlockRows) : N;
  const int nT = (kv_end + kTileKeys - 1) / kTileKeys;

  // Start the first two tiles before anything else.
  issue_tile(k_rsrc, v_rsrc, smem, 0, wave, lane);
  if (nT > 1) issue_tile(k_rsrc, v_rsrc, smem + kTileBytes, kTileKeys, wave, lane);

  WaveState w;
#pragma unroll
  for (int c = 0; c < 4; ++c)
    w.qop[c] = __builtin_bit_cast(bf16x8, buf_load16(q_rsrc, qrow * kKRowBytes + 32 * c + 16 * h));

  // K A-operand, key half kh, d chunk c: row 32kh + r32, logical 16-B chunk 2c + h.
#pragma unroll
  for (int kh = 0; kh < 2; ++kh)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int row = 32 * kh + r32;
      w.koff[kh][c] = row * kKRowBytes + (((2 * c + h) ^ swz_k(row)) << 4);
    }
  // V^T operand, d tile dt, run s of 4 keys: source lane (group g = lane/16, j = lane%16)
  // reads V[16*c4 + 8s + 4(g/2) + j/4][32dt + 16(g%2) + 4(j%4) .. +3]; the c4 term is an
  // immediate offset of 16 rows.
  {
    const int g = lane >> 4, jj = lane & 15;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int sr = 0; sr < 2; ++sr) {
        const int row = 8 * sr + 4 * (g >> 1) + (jj >> 2);
        const int d0 = 32 * dt + 16 * (g & 1) + 4 * (jj & 3);
        w.voff[dt][sr] = kHalfTileBytes + row * kKRowBytes + (((d0 >> 3) ^ swz_v(row)) << 4) +
                         (d0 & 7) * 2;
      }
  }
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    w.o0[t] = 0.f;
    w.o1[t] = 0.f;
  }
  w.m_run = -INFINITY;
  w.l_run = 0.f;

  // Last visible key of this lane's row, for the element mask.
  const int last_key = causal ? min(qrow, N - 1) : N - 1;

  for (int j = 0; j < nT; j += kStages) {
    pipeline_step<0>(w, smem, j, nT, k_rsrc, v_rsrc, wave, lane, q0, N, causal, last_key, h, scale_log2);
    if (j + 1 >= nT) break;
    pipeline_step<1>(w, smem, j + 1, nT, k_rsrc, v_rsrc, wave, lane, q0, N, causal, last_key, h, scale_log2);
    if (j + 2 >= nT) break;
    pipeline_step<2>(w, smem, j + 2, nT, k_rsrc, v_rsrc, wave, lane, q0, N, causal, last_key, h, scale_log2);
  }

  if (qrow < N) {
    const float inv_l = 1.0f / w.l_run;
    __bf16* orow = O + head_off + (size_t)qrow * kD;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      bf16x4 lo4, hi4;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        lo4[r] = (__bf16)(w.o0[4 * g + r] * inv_l);
        hi4[r] = (__bf16)(w.o1[4 * g + r] * inv_l);
      }
      *reinterpret_cast<bf16x4*>(orow + 8 * g + 4 * h) = lo4;
      *reinterpret_cast<bf16x4*>(orow + 32 + 8 * g + 4 * h) = hi4;
    }
    if (LSE != nullptr && h == 0) {
      LSE[(size_t)bh * N + qrow] = (w.m_run + __builtin_amdgcn_logf(w.l_run)) * kLn2;
    }
  }
}

// ---------------------------------------------------------------------------------------
// Host side: argument validation, cached device properties, launch.

struct DeviceInfo {
  int cu_count = 0;
  int sclk_mhz = 0;
  char arch[64] = {0};
  int status = 0;
};

constexpr int kMaxDevices = 64;
static std::once_flag g_dev_once[kMaxDevices];
static DeviceInfo g_dev_info[kMaxDevices];

// Argument checks, in this order: sizes and flags first, then - only for a non-empty
// problem - pointers.  An empty tensor may legitimately have a null data pointer
// (torch gives numel()==0 tensors address 0), so B, H or N == 0 succeeds with no launch.
static int validate(const void* q, const void* k, const void* v, const void* o, const float* lse,
                    int B, int H, int N, int D, float scale, int causal) {
  if (B < 0 || H < 0 || N < 0) return TFGFA_ERR_BAD_SHAPE;
  if (D != kD) return TFGFA_ERR_HEAD_DIM;
  if (!(scale > 0.f) || !isfinite(scale)) return TFGFA_ERR_SCALE;
  if (causal != 0 && causal != 1) return TFGFA_ERR_CAUSAL_FLAG;
  if (B == 0 || H == 0 || N == 0) return TFGFA_OK;
  if (q == nullptr || k == nullptr || v == nullptr || o == nullptr) return TFGFA_ERR_NULL_POINTER;
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)o) & 15u) return TFGFA_ERR_ALIGNMENT;
  if (((uintptr_t)lse) & 3u) return TFGFA_ERR_ALIGNMENT;
  const long long bh = (long long)B * H;
  const long long nqb = ((long long)N + kBlockRows - 1) / kBlockRows;
  if (bh > INT32_MAX || bh * nqb > INT32_MAX) return TFGFA_ERR_TOO_LARGE;
  // Per-head byte offsets (row * 128 B) are 32-bit buffer offsets.
  if (((long long)N + kBlockRows) * kKRowBytes > INT32_MAX) return TFGFA_ERR_TOO_LARGE;
  return TFGFA_OK;
}

}  // namespace tfgfa

extern "C" int tfgfa_fwd_bf16(const void* q, const void* k, const void* v, void* o, float* lse,
                              int B, int H, int N, int D, float softmax_scale, int causal,
                              void* hip_stream) {
  using namespace tfgfa;
  const int st = validate(q, k, v, o, lse, B, H, N, D, softmax_scale, causal);
  if (st != TFGFA_OK) return st;
  if (B == 0 || H == 0 || N == 0) return TFGFA_OK;

  const int BH = B * H;
  const int nQB = (N + kBlockRows - 1) / kBlockRows;
  const float scale_log2 = softmax_scale * kLog2e;
  hipLaunchKernelGGL(fwd_kernel, dim3(BH * nQB), dim3(kThreads), 0, (hipStream_t)hip_stream,
                     static_cast<const __bf16*>(q), static_cast<const __bf16*>(k),
                     static_cast<const __bf16*>(v), static_cast<__bf16*>(o), lse, BH, N, nQB,
                     scale_log2, causal);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? TFGFA_OK : -(int)e;
}

extern "C" const char* tfgfa_strerror(int status) {
  switch (status) {
    case TFGFA_OK: return "success";
    case TFGFA_ERR_NULL_POINTER: return "null tensor pointer (q, k, v and o are required)";
    case TFGFA_ERR_BAD_SHAPE: return "negative batch, head or sequence size";
    case TFGFA_ERR_HEAD_DIM: return "unsupported head dimension (only 64 is compiled)";
    case TFGFA_ERR_SCALE: return "softmax_scale must be finite and > 0";
    case TFGFA_ERR_CAUSAL_FLAG: return "causal flag must be 0 or 1";
    case TFGFA_ERR_TOO_LARGE: return "problem exceeds the launch limits (B*H*ceil(N/128) < 2^31)";
    case TFGFA_ERR_ALIGNMENT: return "misaligned pointer (q/k/v/o need 16 B, lse 4 B)";
    default: break;
  }
  if (status < 0) return hipGetErrorString((hipError_t)(-status));
  return "unknown tfgfa status";
}

extern "C" int tfgfa_device_info(int* cu_count, int* sclk_mhz, char* arch, int arch_len) {
  using namespace tfgfa;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return -(int)e;
  if (dev < 0 || dev >= kMaxDevices) return TFGFA_ERR_TOO_LARGE;
  std::call_once(g_dev_once[dev], [dev]() {
    hipDeviceProp_t prop;
    const hipError_t pe = hipGetDeviceProperties(&prop, dev);
    if (pe != hipSuccess) {
      g_dev_info[dev].status = -(int)pe;
      return;
    }
    g_dev_info[dev].cu_count = prop.multiProcessorCount;
    g_dev_info[dev].sclk_mhz = prop.clockRate / 1000;
    strncpy(g_dev_info[dev].arch, prop.gcnArchName, sizeof(g_dev_info[dev].arch) - 1);
  });
  const DeviceInfo& di = g_dev_info[dev];
  if (di.status != 0) return di.status;
  if (cu_count) *cu_count = di.cu_count;
  if (sclk_mhz) *sclk_mhz = di.sclk_mhz;
  if (arch && arch_len > 0) {
    strncpy(arch, di.arch, (size_t)arch_len - 1);
    arch[arch_len - 1] = '\0';
  }
  return TFGFA_OK;
}

extern "C" int tfgfa_abi_version(void) { return TFGFA_ABI_VERSION; }
