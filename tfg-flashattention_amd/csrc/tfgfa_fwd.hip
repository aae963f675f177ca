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
//   32 query rows.  Keys are staged in 64-key tiles but processed in 32-key halves, which line
//   up with the wave's 32 rows: a half is either wholly visible, wholly above the causal
//   diagonal (never computed) or the single diagonal block (element mask).  Tiles wholly above
//   the diagonal of the whole block are never loaded.  Workgroups are issued heaviest query
//   block first.
//
// Per-wave software pipeline (32-key halves u = 0, 1, ...)
//   half-step u:  O += V_{u-1} P_{u-1}   interleaved with   P_u = exp2(S_u - m)
//                 (move the offset m if some score passed it by the margin: rare branch)
//                 S_{u+1} = K_{u+1} Q^T  interleaved with   row sums of P_u, P_u to bf16/fp16
//   The steady half-step is a fixed sequence of chunks (one MFMA, the next operand read, a
//   share of the VALU work) held in order by scheduling fences: a wave's VALU work overlaps
//   its own in-flight MFMAs.  The S double buffer is 2 x 16 registers; 168 VGPRs keep three
//   waves per SIMD at head dim 64.
//
// Memory pipeline
//   K and V tiles go from HBM straight into LDS (buffer_load_dwordx4 ... lds: each lane's
//   16 B land at LDS base + 16*lane), no registers or VALU spent on staging.  A ring of 2
//   (head dim 64) or 3 (head dim 128) K slots and a ring of 2 V slots.  Tile step j: (3 K
//   slots: issue K_{j+2}); half-step 2j (uses K_j, V_{j-1}); wait for this wave's loads of
//   K_{j+1} and V_j and barrier; issue V_{j+1} into V_{j-1}'s slot (2 K slots: and K_{j+2}
//   into K_j's); half-step 2j+1 (uses K_{j+1}, V_j).  The barrier also proves every wave has
//   finished with the slots refilled after it.  At head dim 64 the prologue also moves the
//   wave's Q rows through LDS, so the first S waits for Q and K_0 only (K_1 and V_0 are waited
//   for in tile step 0).
//   Loads past the sequence end return zero (buffer range check): the zero-fill of partial
//   tiles.
//
// Epilogue
//   O is normalised, written to LDS (head dim 64: the wave's Q stage; head dim 128: a share of
//   the ring after a final barrier) and read back so that each lane stores 16 B of one row:
//   every store instruction writes whole 128-B (or 256-B) rows, non-temporally.  Storing the
//   O^T accumulators directly wrote 16 B of each of 32 rows per instruction.
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
//   16-B chunk c of row r is stored at chunk c ^ swz(r).  K: swz = (r ^ ((r >> 3) & 3)) & 7
//   makes any 8 (or 16) consecutive rows of one logical chunk hit distinct banks for the
//   ds_read_b128 A-operand reads, and is the same for rows r and r + 32, so the two key halves
//   of a tile differ by an immediate offset.  V: swz = 2*(r & 3) makes the 4-row x 32-B footprint of a transposing read
//   group (and of two groups side by side) hit distinct banks.
//
// Softmax runs in the exp2 domain: scores are scaled by scale*log2(e) inside one FMA; the
// offset m and the sums l_run (fp32 probabilities) and l_p (rounded probabilities) are
// per-lane registers; O = (P.V) / l_p and LSE = (m + log2 l_run) * ln 2.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <string.h>

#include <mutex>
#include <type_traits>

#include "tfgfa.h"

namespace tfgfa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kDHalf = 64;                  // head dims per LDS tile layout ("dim half")
constexpr int kWaves = 4;                   // waves per workgroup
constexpr int kThreads = kWaves * 64;       // 256
constexpr int kWaveRows = 32;               // query rows per wave (one MFMA column block)
constexpr int kBlockRows = kWaves * kWaveRows;  // 128 query rows per workgroup
constexpr int kTileKeys = 64;               // keys per K/V tile
constexpr int kKRowBytes = kDHalf * 2;      // 128 B per key row of one dim half in LDS
constexpr int kHalfTileBytes = kTileKeys * kKRowBytes;  // 8 KiB (K or V, one dim half)
constexpr int kMaxD = 128;
// A buffer offset past any num_records built here (those stay below 2^31 - 2^24): the load
// returns zero without a memory access.  Used for head dims past D when D < the tile's dims.
constexpr int kOutOfRange = 0x7FFFFFF0;

// The exp2 offset m of a row moves (to the row's exact running max, rescaling O and the sums)
// only when the probabilities grow too large: for bf16 in a full half-step, when a lane's running
// sum of its rounded probabilities would pass 2^64; otherwise (fp16, and a wave's last
// half-step), when some score exceeds m by more than the type's margin (60 / 15 log2 units).
// So P stays bounded and the rescale is rare.  For bf16 a lane's probabilities sum to at most
// 2^64 through the full half-steps and its last half adds at most 16 * 2^60 = 2^64, so each P.V
// accumulator stays below 2^66 * max|V|.  O is normalised by l_p, the sum of the probabilities
// *as rounded* for the P.V MFMA, so the rounding of a dominant probability cancels between O's
// numerator and denominator; the LSE uses l_run, the fp32 sum of the unrounded ones.

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Element type traits: the 16-bit type of Q, K, V, O and of the P operand, its 8-vector, and the
// matching 32x32x16 MFMA (fp32 accumulate).
template <typename T>
struct Elem;
template <>
struct Elem<__bf16> {
  typedef bf16x8 v8;
  typedef bf16x4 v4;
  static __device__ __forceinline__ f32x16 mfma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  // Offset margin (log2 units) of the lane-max check of a wave's last half: P <= 2^60, so the
  // lane's 16 probabilities of that half sum to at most 2^64.
  static constexpr float kMargin = 60.0f;
  // Bound on a lane's running probability sum in the fused half-step's offset check (every P
  // so far is at most the sum).
  static constexpr float kSumBound = 0x1p64f;
  // acc + the sum of the 8 elements of p (exact products by 1, fp32 accumulation).
  static __device__ __forceinline__ float sum8(v8 p, float acc) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p, p, 0, 1), one, acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p, p, 2, 3), one, acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p, p, 4, 5), one, acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p, p, 6, 7), one, acc, false);
    return acc;
  }
};
template <>
struct Elem<_Float16> {
  typedef f16x8 v8;
  typedef f16x4 v4;
  static __device__ __forceinline__ f32x16 mfma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  // Offset margin of the lane-max check of a wave's last half: P <= 2^15 stays inside fp16's
  // range (65504).
  static constexpr float kMargin = 15.0f;
  // Bound of the fused half-step's sum check: the largest finite float.  The conversion to fp16
  // gives +inf for a P above fp16's range, so the rounded sum exceeds the bound (is +inf or a
  // NaN) exactly when some rounded P is not finite; every finite one is at most 65504, which
  // keeps l_p and |O| / max|V| below 2^16 times the number of keys.  Measured against checking
  // the lane max of the scores against the margin on every half-step (the rounded sum is
  // computed anyway, the lane max is ~10 more VALU instructions), interleaved, µs: B1 H16 N8192
  // 171.7 -> 165.9, B8 H16 N1024 d = 128 54.7 -> 54.0, B8 H25 N1024 (sigma = 3, O + LSE)
  // 50.2 -> 49.6.
  static constexpr float kSumBound = 0x1.fffffep127f;
  static __device__ __forceinline__ float sum8(v8 p, float acc) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 0, 1), one, acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 2, 3), one, acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 4, 5), one, acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 6, 7), one, acc, false);
    return acc;
  }
};

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

__device__ __forceinline__ int swz_k(int row) { return (row ^ ((row >> 3) & 3)) & 7; }
__device__ __forceinline__ int swz_v(int row) { return (row & 3) << 1; }

// Buffer descriptor over one head's N rows (row r at byte r * row_bytes; row_bytes = 2 * D for
// a contiguous head), as four SGPRs for the loads issued from inline assembly: base address,
// stride 0, num_records = N * row_bytes, format word 0x20000 (the layout
// __builtin_amdgcn_make_buffer_rsrc builds for the Q loads).  A raw buffer load whose byte
// offset is at or past num_records returns zero: that is the zero-fill of tiles and query
// blocks past the sequence end (row N starts exactly at num_records: rows are at least 2D
// bytes apart and a lane never reads past byte 2D of a row).  The whole offset is kept in the
// VGPR operand so the range check covers all of it.
typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ i32x4 head_desc(const void* base, int N, int row_bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  i32x4 d;
  d[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  d[1] = __builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
  d[2] = N * row_bytes;
  d[3] = 0x00020000;
  return d;
}

// One 1-KiB HBM -> LDS transfer: lane i's 16 B (global byte offset `voff` in the buffer) land at
// LDS byte address lds_base + 16*i.  Issued from inline assembly so that the compiler does not
// track it: it would otherwise wait for every outstanding transfer before LDS reads it cannot
// prove disjoint (it loses that proof at control-flow joins).  The only waits on these
// transfers are the explicit vmcnt waits of the pipeline.
// The transfer takes its LDS address from M0, a register the compiler reserves (a clobber of it
// is not honoured).  So the statement saves M0 in a scalar register of its own, sets it, issues
// the load and puts the saved value back: whatever the compiler keeps in M0 is unchanged after
// the statement.  The s_nop is the one wait state GFX9 needs between an SALU write of M0 and an
// LDS DMA that reads it.
__device__ __forceinline__ void lds_transfer(i32x4 desc, uint32_t lds_base, int voff) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds_base), "v"(voff), "s"(desc)
      : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const unsigned char* p) {
  return (uint32_t)(uintptr_t)(const lds_void*)p;
}

// Compile-time shape of one kernel instance: head dims kD (64 or 128, = kDH dim halves of 64),
// element type T, and kMaskD: the actual head dim D may be below kD (a multiple of 8); 16-B
// chunks of dims >= D load zeros and are not stored.  kLse: the LSE is written, so the fp32
// sum l_run is kept (without it only l_p, which normalises O, is summed).
template <int kD_, typename T_, bool kMaskD_, bool kLse_ = true>
struct Shape {
  static constexpr int kD = kD_;
  static constexpr bool kLse = kLse_;
  static constexpr int kDH = kD_ / kDHalf;
  static constexpr bool kMaskD = kMaskD_;
  typedef T_ T;
  static constexpr int kLoadsPerWave = 4 * kDH;  // transfers per tile step per wave (K and V)
  // K ring slots.  2: K_{j+2} is issued after tile step j's barrier, into the slot of K_j (last
  // read by half-step 2j, before the barrier), and has two half-steps to land.  3: K_{j+2} is
  // issued at the start of step j, into the slot of K_{j-1}, and has three.  Head dim 64 uses 2
  // (as fast, measured, and it leaves LDS for the Q stage); head dim 128 uses 3: 2 slots (a third
  // of the code, 64 KiB of LDS) measured 0.3-2.4% slower at d = 128, 120, 112, 72 and 96 (B1 H16
  // N8192), faster only at B8 H25 N1024 d = 96 (2.7%).
  static constexpr int kKSlots = kD_ == 128 ? 3 : 2;
  // V ring: 2 slots; V_{j+1} is issued after step j's barrier, into the slot of V_{j-1} (read by
  // half-step 2j, before the barrier).
  static constexpr int kVSlots = 2;
  // Tile steps after which the K and V slot assignments repeat.
  static constexpr int kPeriod = kKSlots == 3 ? 6 : 2;
  // Q reaches its registers through LDS (a 4-KiB stage per wave): the loads are LDS transfers
  // that the compiler does not track, so the prologue waits for Q and K_0 only.  Head dim 64
  // (48 KiB of LDS per workgroup with the rings, three workgroups per CU); head dim 128 loads Q
  // into registers and waits for the whole prologue (its rings take 80 KiB).
  static constexpr bool kQStage = kD_ == 64;
  static_assert(kD_ == 64 || kD_ == 128, "compiled head dims");
};

// This wave's share of one K (or V) tile: rows [8*(2w), 8*(2w+2)) of each dim half as two
// 1-KiB LDS blocks per dim half (dim half dh at byte dh * 8 KiB of the slot).  Lane i of a block
// fills physical chunk i%8 of row i/8, so it fetches the logical chunk that the swizzle maps
// there: head dims 64*dh + 8*chunk .. +7, i.e. row bytes 128*dh + 16*chunk.
// The lane's byte offset within a tile (from the tile's first row) is the same for every tile,
// so it is computed once (tile_offsets); per tile only the descriptor moves (tile_desc), in
// scalar registers, and the transfers take no VALU work.
template <class Sh>
__device__ __forceinline__ void tile_offsets(int (*koff)[2], int (*voff)[2], int k_row_bytes,
                                             int v_row_bytes, int wave, int lane, int d_chunks) {
#pragma unroll
  for (int dh = 0; dh < Sh::kDH; ++dh)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = (2 * wave + i) * 8 + (lane >> 3);
      const int kc = 8 * dh + ((lane & 7) ^ swz_k(row));  // 16-B chunk of the row in memory
      const int vc = 8 * dh + ((lane & 7) ^ swz_v(row));
      int ko = row * k_row_bytes + (kc << 4);
      int vo = row * v_row_bytes + (vc << 4);
      if (Sh::kMaskD) {
        ko = kc < d_chunks ? ko : kOutOfRange;
        vo = vc < d_chunks ? vo : kOutOfRange;
      }
      koff[dh][i] = ko;
      voff[dh][i] = vo;
    }
}

// The head's descriptor moved to row k0: base + k0 rows, num_records reduced by as much, so a
// row at or past the sequence end still reads zero.  k0 < N for every tile issued.
__device__ __forceinline__ i32x4 tile_desc(i32x4 desc, int k0, int row_bytes) {
  const uint32_t adv = (uint32_t)(k0 * row_bytes);
  const uint64_t base = ((uint64_t)(uint32_t)desc[1] << 32 | (uint32_t)desc[0]) + adv;
  i32x4 d;
  d[0] = (int)(uint32_t)base;
  d[1] = (int)(uint32_t)(base >> 32);
  d[2] = desc[2] - (int)adv;
  d[3] = desc[3];
  return d;
}

template <class Sh>
__device__ __forceinline__ void issue_tile(i32x4 desc, int row_bytes, unsigned char* dst, int k0,
                                           int wave, const int (*off)[2]) {
  const i32x4 d = tile_desc(desc, k0, row_bytes);
#pragma unroll
  for (int dh = 0; dh < Sh::kDH; ++dh)
#pragma unroll
    for (int i = 0; i < 2; ++i)
      lds_transfer(d, lds_addr(dst + dh * kHalfTileBytes + (2 * wave + i) * 1024), off[dh][i]);
}

// The workgroup's Q stage (head dim 64): 4 KiB of LDS per wave, allocated only by the instances
// that call this.
template <class Sh>
__device__ __forceinline__ unsigned char* q_stage() {
  __shared__ __attribute__((aligned(1024))) unsigned char qst[kBlockRows * kKRowBytes];
  return qst;
}

// This wave's 32 query rows, from the descriptor's first row, into its 4-KiB LDS stage (head
// dim 64): row r at byte 128 r, logical 16-B chunk c (head dims 8c .. 8c+7) at physical chunk
// c ^ swz_k(r), so the 8 (or 16) consecutive rows of one ds_read_b128 hit distinct banks.  Four
// 1-KiB transfers; rows past the sequence end read zero.
template <class Sh>
__device__ __forceinline__ void issue_q_stage(i32x4 qdesc, int row_bytes, unsigned char* dst,
                                              int d_chunks) {
  static_assert(Sh::kDH == 1, "the Q stage holds 128-B rows");
  int lane;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane));
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int row = 8 * t + (lane >> 3);
    const int lc = (lane & 7) ^ swz_k(row);
    int off = row * row_bytes + (lc << 4);
    if (Sh::kMaskD) off = lc < d_chunks ? off : kOutOfRange;
    lds_transfer(qdesc, lds_addr(dst + t * 1024), off);
  }
}

// Workgroup barrier that is also a compiler memory barrier: no LDS access moves across it (the
// s_barrier builtin alone is not a memory operation for the optimizer), and unlike
// __syncthreads() it adds no wait for outstanding vector memory loads, which would drain the
// load pipeline.  The only LDS writes are the buffer_load ... lds transfers, completed by the
// explicit vmcnt waits before each barrier.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Workgroup barrier after this wave's own LDS writes (ds_write) and reads: s_barrier does not
// wait for the wave's outstanding LDS operations, so they are waited for first; after it,
// every wave sees the writes of every other.
__device__ __forceinline__ void lds_write_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// LDS: a ring of Shape::kKSlots K tiles and a ring of 2 V tiles, each slot kDH dim halves of
// 8 KiB.
struct Lds {
  unsigned char* k[3];
  unsigned char* v[2];
};

// Per-wave state carried across half-steps.
template <class Sh>
struct WaveState {
  typedef typename Elem<typename Sh::T>::v8 v8;
  v8 qop[4 * Sh::kDH];   // Q^T operand: Q[qrow][16c + 8h .. +7]
  f32x16 o[2 * Sh::kDH]; // O^T accumulators: o[t] holds d = 32t .. 32t+31
  f32x16 s;              // S^T of the half being softmaxed: register t = key 8(t/4) + 4h + t%4
  v8 pb[2];              // P^T of the previous half, waiting for its P.V
  float m_run;           // exp2 offset (a running max of scale*log2e*s, moved lazily)
  float thr;             // raw score above which the offset has to move: (m_run + margin) / (scale*log2e)
  float l_run;           // this lane's running sum of exp2(scale*log2e*s - m_run) (fp32, for the LSE)
  float l_p;             // this lane's running sum of the same probabilities rounded to T (for O)
  int koff[4];           // K A-operand LDS offsets (within a K dim half, key half 0)
  int voff[2][2];        // V^T transposing-read LDS offsets (within a V dim half, keys 0..15)
};

// S^T = K Q^T for key half kHalf of the tile in K slot kSlot (4 MFMAs per dim half; dim half dh
// at byte dh * kDhBytes of the slot).
template <class Sh, int kSlot, int kHalf, int kDhBytes = kHalfTileBytes>
__device__ __forceinline__ f32x16 qk_half(const WaveState<Sh>& w, const Lds& lds) {
  typedef typename Elem<typename Sh::T>::v8 v8;
  f32x16 acc;
#pragma unroll
  for (int t = 0; t < 16; ++t) acc[t] = 0.f;
#pragma unroll
  for (int dh = 0; dh < Sh::kDH; ++dh) {
    const unsigned char* kt = lds.k[kSlot] + dh * kDhBytes + kHalf * 32 * kKRowBytes;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const v8 a = *reinterpret_cast<const v8*>(kt + w.koff[c]);
      acc = Elem<typename Sh::T>::mfma(a, w.qop[4 * dh + c], acc);
    }
  }
  return acc;
}

// O^T += V^T P^T for key half kHalf of the tile in V slot kSlot, with P^T = w.pb (4 MFMAs per
// dim half).  Element e of chunk cc in lane half h is key 16*cc + 8*(e/4) + 4*h + e%4 of the
// key half: two transposing reads of 4 keys each.  Dim half dh at byte dh * kDhBytes of the slot.
template <class Sh, int kSlot, int kHalf, int kDhBytes = kHalfTileBytes>
__device__ __forceinline__ void pv_half(WaveState<Sh>& w, const Lds& lds) {
  typedef typename Elem<typename Sh::T>::v8 v8;
#pragma unroll
  for (int dh = 0; dh < Sh::kDH; ++dh) {
    const unsigned char* vt = lds.v[kSlot] + dh * kDhBytes + kHalf * 32 * kKRowBytes;
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(vt + w.voff[dt][0] + cc * 16 * kKRowBytes));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(vt + w.voff[dt][1] + cc * 16 * kKRowBytes));
        const v8 va = __builtin_bit_cast(v8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        w.o[2 * dh + dt] = Elem<typename Sh::T>::mfma(va, w.pb[cc], w.o[2 * dh + dt]);
      }
    }
  }
}

// Masks w.s past the last visible key; lim is the lane's last visible key relative to the
// half's first key + 4h.
template <class Sh>
__device__ __forceinline__ void mask_half(WaveState<Sh>& w, int lim) {
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    const int kk = 8 * (t >> 2) + (t & 3);
    w.s[t] = kk > lim ? -INFINITY : w.s[t];
  }
}

// Max of this lane's 16 raw scores.
template <class Sh>
__device__ __forceinline__ float lane_max(const WaveState<Sh>& w) {
  float mx = fmaxf(w.s[0], fmaxf(w.s[1], w.s[2]));
#pragma unroll
  for (int t = 3; t < 15; t += 2) mx = fmaxf(fmaxf(mx, w.s[t]), w.s[t + 1]);
  return fmaxf(mx, w.s[15]);
}

// Moves the exp2 offset of every row to its exact running max, rescaling O and the sums, when
// some lane's score exceeds its row's offset by more than the margin (wave-uniform branch, taken
// at a wave's first half and then rarely).  Every computed half has an unmasked key in every
// row (it starts at or below the wave's first row), so the pair max is finite and the first
// half always moves m_run off -inf.
template <class Sh>
__device__ __forceinline__ void move_offset(WaveState<Sh>& w, float mx, float scale_log2,
                                            float inv_scale_log2) {
  if (__builtin_amdgcn_ballot_w64(mx > w.thr) != 0) {
    const float m_new = fmaxf(w.m_run, pair_max(mx) * scale_log2);
    const float alpha = __builtin_amdgcn_exp2f(w.m_run - m_new);
    w.m_run = m_new;
    w.thr = (m_new + Elem<typename Sh::T>::kMargin) * inv_scale_log2;
    if constexpr (Sh::kLse) w.l_run *= alpha;
    w.l_p *= alpha;
#pragma unroll
    for (int i = 0; i < 2 * Sh::kDH; ++i)
#pragma unroll
      for (int t = 0; t < 16; ++t) w.o[i][t] *= alpha;
  }
}

// Sum of the probabilities p into l_run, p rounded to the element type into w.pb (chunk cc =
// keys 16cc .. 16cc+15 of the half: registers 8cc .. 8cc+7), the sum of the rounded values
// into l_p.
template <class Sh, class P>
__device__ __forceinline__ void sum_convert(WaveState<Sh>& w, const P& p) {
  typedef typename Sh::T T;
  if constexpr (Sh::kLse) {
    float ps0 = p[0], ps1 = p[1];
#pragma unroll
    for (int t = 2; t < 16; t += 2) {
      ps0 += p[t];
      ps1 += p[t + 1];
    }
    w.l_run += ps0 + ps1;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    w.pb[0][e] = (T)p[e];
    w.pb[1][e] = (T)p[8 + e];
  }
  w.l_p = Elem<T>::sum8(w.pb[1], Elem<T>::sum8(w.pb[0], w.l_p));
}

// P = exp2(scale*log2e*s - m_run) in fp32 (in place), then sum_convert.
template <class Sh>
__device__ __forceinline__ void exp_half(WaveState<Sh>& w, float scale_log2) {
  const float neg_m = -w.m_run;
#pragma unroll
  for (int t = 0; t < 16; ++t) w.s[t] = __builtin_amdgcn_exp2f(fmaf(w.s[t], scale_log2, neg_m));
  sum_convert(w, w.s);
}

template <class Sh, int kVs, int kVh>
__device__ __forceinline__ typename Elem<typename Sh::T>::v8 v_operand(const WaveState<Sh>& w,
                                                                      const Lds& lds, int i) {
  typedef typename Elem<typename Sh::T>::v8 v8;
  const int dh = i >> 2, cc = (i >> 1) & 1, dt = i & 1;
  const unsigned char* vt =
      lds.v[kVs] + dh * kHalfTileBytes + kVh * 32 * kKRowBytes + cc * 16 * kKRowBytes;
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(vt + w.voff[dt][0]));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(vt + w.voff[dt][1]));
  return __builtin_bit_cast(v8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

template <class Sh, int kKs, int kKh>
__device__ __forceinline__ typename Elem<typename Sh::T>::v8 k_operand(const WaveState<Sh>& w,
                                                                      const Lds& lds, int i) {
  typedef typename Elem<typename Sh::T>::v8 v8;
  const int dh = i >> 2, c = i & 3;
  const unsigned char* kt = lds.k[kKs] + dh * kHalfTileBytes + kKh * 32 * kKRowBytes;
  return *reinterpret_cast<const v8*>(kt + w.koff[c]);
}

#define TFGFA_FENCE() __builtin_amdgcn_sched_barrier(0)

// A full half-step u as a fixed sequence of chunks, each MFMA followed by a share of the VALU
// work that does not depend on it (a wave's VALU work overlaps its own in-flight MFMAs):
//   chunk 0          V^T operands of the first two P.V MFMAs
//   chunks 1..kPv    MFMA i of O += V_{u-1} P_{u-1}, the next operand read, a share of
//                    P_u = exp2(scale*log2e*S_u - m_run)
//   chunks kPv+1..   MFMA i of S_{u+1} = K_{u+1} Q^T, the next operand read, a share of
//                    the sums of P_u and its conversion to the element type
// The offset check reads the lane's running sum l_p with this half's probabilities, as rounded
// to the element type, added.  bf16: a rounded P above 2^64 makes that sum exceed the bound (an
// overflow gives +inf, a -inf offset on a wave's first half gives +inf or NaN), so a sum above
// the bound, or not a number, takes the rare branch: move the offset to the rows' exact running
// max, rescale O and the sums, recompute P_u.  A sum above the bound without any single P above
// it moves the offset early, which is harmless (after a move every P is at most 1, so l_p stays
// below the number of keys).  So l_p, and with it every P and |O| / max|V|, stays at most 2^64.
// fp16: the bound is the largest finite float, exceeded exactly when a rounded P is +inf (above
// fp16's range) or a NaN, so every P that reaches an MFMA is finite.
template <class Sh, int kVs, int kVh, int kKs, int kKh, bool kPV = true>
__device__ __forceinline__ void fused_step(WaveState<Sh>& w, const Lds& lds, float scale_log2,
                                           float inv_scale_log2) {
  typedef typename Sh::T T;
  typedef typename Elem<T>::v8 v8;
  constexpr int kPv = 4 * Sh::kDH;
  constexpr int kS = 4 * Sh::kDH;
  constexpr float kSumBound = Elem<T>::kSumBound;
  v8 vop[2];
  if constexpr (kPV) {
    vop[0] = v_operand<Sh, kVs, kVh>(w, lds, 0);
    vop[1] = v_operand<Sh, kVs, kVh>(w, lds, 1);
  }
  TFGFA_FENCE();
  const float neg_m = -w.m_run;
  float p[16];
  v8 kop[2];
#pragma unroll
  for (int i = 0; i < kPv; ++i) {
    const int dh = i >> 2, cc = (i >> 1) & 1, dt = i & 1;
    if constexpr (kPV) w.o[2 * dh + dt] = Elem<T>::mfma(vop[i & 1], w.pb[cc], w.o[2 * dh + dt]);
    if (i + 2 < kPv) {
      if constexpr (kPV) vop[i & 1] = v_operand<Sh, kVs, kVh>(w, lds, i + 2);
    } else {
      kop[i + 2 - kPv] = k_operand<Sh, kKs, kKh>(w, lds, i + 2 - kPv);
    }
#pragma unroll
    for (int t = 16 * i / kPv; t < 16 * (i + 1) / kPv; ++t)
      p[t] = __builtin_amdgcn_exp2f(fmaf(w.s[t], scale_log2, neg_m));
    // Computed here, in this chunk, even though the rare branch recomputes them.
#pragma unroll
    for (int t = 16 * i / kPv; t < 16 * (i + 1) / kPv; ++t) asm volatile("" : "+v"(p[t]));
    TFGFA_FENCE();
  }
  f32x16 acc;
#pragma unroll
  for (int t = 0; t < 16; ++t) acc[t] = 0.f;
  // Chunk 0 converts P_u to the element type, chunk 1 sums the rounded values, checks the
  // offset on that sum and adds it to l_p, chunk 2 adds the fp32 sum to l_run (LSE only).  Both
  // instances (with and without the LSE) take the same branch decisions, so their O agree bit
  // for bit.
  auto convert = [&w](const float* q) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      w.pb[0][e] = (T)q[e];
      w.pb[1][e] = (T)q[8 + e];
    }
  };
#pragma unroll
  for (int i = 0; i < kS; ++i) {
    acc = Elem<T>::mfma(kop[i & 1], w.qop[i], acc);
    if (i + 2 < kS) kop[i & 1] = k_operand<Sh, kKs, kKh>(w, lds, i + 2);
    if (i == 0) {
      convert(p);
      asm volatile("" : "+v"(w.pb[0]), "+v"(w.pb[1]));
    } else if (i == 1) {
      // The running sum with this half's rounded probabilities added (one of the two dot2
      // chains starts from l_p).
      float hs = Elem<T>::sum8(w.pb[0], w.l_p) + Elem<T>::sum8(w.pb[1], 0.f);
      // As unsigned integers, the bits of a sum >= +0 exceed those of the bound exactly when
      // the sum does, is +inf or is a NaN (the device pass assumes no NaN in float compares).
      if (__builtin_amdgcn_ballot_w64(__float_as_uint(hs) > __float_as_uint(kSumBound)) != 0) {
        const float mx = lane_max(w);
        const float m_new = fmaxf(w.m_run, pair_max(mx) * scale_log2);
        const float alpha = __builtin_amdgcn_exp2f(w.m_run - m_new);
        w.m_run = m_new;
        w.thr = (m_new + Elem<T>::kMargin) * inv_scale_log2;
        if constexpr (Sh::kLse) w.l_run *= alpha;
        w.l_p *= alpha;
#pragma unroll
        for (int j = 0; j < 2 * Sh::kDH; ++j)
#pragma unroll
          for (int t = 0; t < 16; ++t) w.o[j][t] *= alpha;
#pragma unroll
        for (int t = 0; t < 16; ++t) p[t] = __builtin_amdgcn_exp2f(fmaf(w.s[t], scale_log2, -m_new));
        convert(p);
        hs = Elem<T>::sum8(w.pb[0], 0.f) + Elem<T>::sum8(w.pb[1], 0.f);
        hs += w.l_p;  // l_p already rescaled by alpha
      }
      w.l_p = hs;
      asm volatile("" : "+v"(w.l_p));
    } else if (i == 2 && Sh::kLse) {
      float s0 = p[0], s1 = p[1];
#pragma unroll
      for (int t = 2; t < 16; t += 2) {
        s0 += p[t];
        s1 += p[t + 1];
      }
      w.l_run += s0 + s1;
      asm volatile("" : "+v"(w.l_run));
    }
    TFGFA_FENCE();
  }
  w.s = acc;
}

// Loop-invariant inputs of the pipeline.
struct StepArgs {
  i32x4 k_rsrc, v_rsrc;
  int k_row_bytes, v_row_bytes;  // byte distance between consecutive K (V) rows of a head
  int d_chunks;  // 16-B chunks of a row holding head dims < D
  int k_lane[2][2], v_lane[2][2];  // this lane's byte offsets within a K / V tile (tile_offsets)
  int nT;        // 64-key tiles loaded by the workgroup
  int nAct;      // 32-key halves this wave computes (a prefix)
  int nFull;     // halves this wave computes without an element mask (a prefix of the above)
  int wave, lane, h, last_key;
  float scale_log2, inv_scale_log2;
};

// Half-step u: P.V of half u-1 (V slot kVs, half kVh), softmax of half u, S of half u+1 (K
// slot kKs, half kKh).  kSteady: 1 <= u < nAct - 1 is not required, only u < nAct (a full
// half-step) - no early exits, so each MFMA group shares a basic block with independent VALU
// work (P.V with the row max, S_{u+1} with the exponentials):
//  - u = 0 has no P.V before it (kPV = false; the tail path skips it at run time);
//  - S_{u+1} is computed even past the wave's last half (finite, discarded).
// Otherwise (tail): u = nAct is the P.V of the last half only; u > nAct does nothing.
template <class Sh, int kVs, int kVh, int kKs, int kKh, bool kSteady, bool kPV = true>
__device__ __forceinline__ void half_step(WaveState<Sh>& w, const Lds& lds, int u,
                                          const StepArgs& a) {
  if (!kSteady && u > a.nAct) return;
  if (u >= a.nFull && u < a.nAct) mask_half(w, a.last_key - u * 32 - 4 * a.h);
  if (kSteady) {
    fused_step<Sh, kVs, kVh, kKs, kKh, kPV>(w, lds, a.scale_log2, a.inv_scale_log2);
    return;
  }
  if (u > 0) pv_half<Sh, kVs, kVh>(w, lds);
  const float mx = lane_max(w);
  if (!kSteady && u == a.nAct) return;
  move_offset(w, mx, a.scale_log2, a.inv_scale_log2);
  const f32x16 n = qk_half<Sh, kKs, kKh>(w, lds);
  exp_half(w, a.scale_log2);
  w.s = n;
}

// Tile step j (K slot kKs = j % kKSlots, V slot kVs = j % 2): (3 K slots: issue K_{j+2});
// half-step 2j; wait for K_{j+1} and V_j; barrier; issue V_{j+1} (2 K slots: and K_{j+2});
// half-step 2j+1.
template <class Sh, int kKs, int kVs, bool kSteady, bool kFirst = false>
__device__ __forceinline__ void tile_step(WaveState<Sh>& w, const Lds& lds, int j,
                                          const StepArgs& a) {
  constexpr int kKN = Sh::kKSlots;
  constexpr int kKNext = (kKs + 1) % kKN;
  constexpr int kKNext2 = (kKs + 2) % kKN;  // K_{j-1}'s slot (3 slots), K_j's (2 slots)
  constexpr int kVOther = kVs ^ 1;          // V_{j-1}, then V_{j+1}
  const bool k2 = j + 2 < a.nT, v1 = j + 1 < a.nT;
  if (kKN == 3 && k2)
    issue_tile<Sh>(a.k_rsrc, a.k_row_bytes, lds.k[kKNext2], (j + 2) * kTileKeys, a.wave,
                   a.k_lane);
  // Half 2j: P.V of half 2j-1 (V_{j-1}, keys 32..63), S of half 2j+1 (K_j, keys 32..63).
  half_step<Sh, kVOther, 1, kKs, 1, kSteady, !kFirst>(w, lds, 2 * j, a);
  // K_{j+1} and V_j were issued by step j-1 (step 0: by the prologue); only K_{j+2}, issued
  // above with a 3-slot K ring, may stay in flight.
  if (kKN == 3 && k2)
    wait_vmcnt<Sh::kLoadsPerWave / 2>();
  else
    wait_vmcnt<0>();
  lds_barrier();
  if (v1)
    issue_tile<Sh>(a.v_rsrc, a.v_row_bytes, lds.v[kVOther], (j + 1) * kTileKeys, a.wave,
                   a.v_lane);
  if (kKN == 2 && k2)
    issue_tile<Sh>(a.k_rsrc, a.k_row_bytes, lds.k[kKNext2], (j + 2) * kTileKeys, a.wave,
                   a.k_lane);
  // Half 2j+1: P.V of half 2j (V_j, keys 0..31), S of half 2j+2 (K_{j+1}, keys 0..31).
  half_step<Sh, kVs, 0, kKNext, 0, kSteady>(w, lds, 2 * j + 1, a);
}

// Tile step j with its slots chosen at run time (j % kPeriod).
template <class Sh, bool kSteady, int kP = 0>
__device__ __forceinline__ void tile_step_at(WaveState<Sh>& w, const Lds& lds, int j,
                                             const StepArgs& a) {
  if constexpr (kP < Sh::kPeriod) {
    if (j % Sh::kPeriod == kP)
      tile_step<Sh, kP % Sh::kKSlots, kP % Sh::kVSlots, kSteady>(w, lds, j, a);
    else
      tile_step_at<Sh, kSteady, kP + 1>(w, lds, j, a);
  }
}

// kPeriod steady tile steps j0 .. j0 + kPeriod - 1 (j0 = kJ0 modulo kPeriod), slots at
// compile time.
template <class Sh, int kJ0 = 0, int kP = 0>
__device__ __forceinline__ void steady_period(WaveState<Sh>& w, const Lds& lds, int j0,
                                              const StepArgs& a) {
  if constexpr (kP < Sh::kPeriod) {
    tile_step<Sh, (kJ0 + kP) % Sh::kKSlots, (kJ0 + kP) % Sh::kVSlots, true>(w, lds, j0 + kP, a);
    steady_period<Sh, kJ0, kP + 1>(w, lds, j0, a);
  }
}

// The steady tile steps j0 .. n - 1 of a partial period (n - j0 < kPeriod, j0 = kJ0 modulo
// kPeriod), slots at compile time.
template <class Sh, int kJ0 = 0, int kP = 0>
__device__ __forceinline__ void steady_rest(WaveState<Sh>& w, const Lds& lds, int j0, int n,
                                            const StepArgs& a) {
  if constexpr (kP + 1 < Sh::kPeriod) {
    if (j0 + kP < n) {
      tile_step<Sh, (kJ0 + kP) % Sh::kKSlots, (kJ0 + kP) % Sh::kVSlots, true>(w, lds, j0 + kP, a);
      steady_rest<Sh, kJ0, kP + 1>(w, lds, j0, n, a);
    }
  }
}

// The epilogue's O store for a wave's 32 rows.  The O^T accumulators give lane (r, h) head dims
// 32i + 8g + 4h .. +3 of row r, so storing them directly writes 16 B of each of 32 rows per
// store instruction.  Instead the normalised rows go through `stage` (32 rows of 2*kD bytes,
// 16-B chunk c of row r at physical chunk c ^ (r % (kD/8)): the 8-B writes of consecutive rows
// and the 16-B reads of one row hit distinct banks), and each lane then stores 16 B of one
// row: kD/8 lanes write a whole row, one store instruction 8 (head dim 64) or 4 (head dim 128)
// whole rows.  Whole-row stores are non-temporal (O is not read again here, and full lines need
// no write combining in the L2).  With masked head dims (D < kD) rows are only partly written,
// and those stores stay ordinary.  The stage is the wave's alone: LDS accesses of one wave
// complete in order, so the reads see the writes without a barrier.
template <class Sh>
__device__ __forceinline__ void store_o(const WaveState<Sh>& w, unsigned char* stage, float inv_l,
                                        int lane, typename Sh::T* ohead, long long row_stride,
                                        int q0, int Nq, int d_chunks) {
  typedef typename Sh::T T;
  typedef typename Elem<T>::v4 v4;
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  constexpr int kChunks = Sh::kD / 8;  // 16-B chunks per row
  constexpr int kRowB = Sh::kD * 2;
  const int r = lane & 31, h = lane >> 5;
#pragma unroll
  for (int i = 0; i < 2 * Sh::kDH; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      // Register 4g + e of tile i holds dim 32i + 8g + 4h + e: chunk 4i + g, bytes 8h .. 8h+7.
      v4 x;
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = (T)(w.o[i][4 * g + e] * inv_l);
      const int c = 4 * i + g;
      *reinterpret_cast<v4*>(stage + r * kRowB + ((c ^ (r % kChunks)) << 4) + 8 * h) = x;
    }
  constexpr int kRowsPerStore = 64 / kChunks;
#pragma unroll
  for (int t = 0; t < 32 / kRowsPerStore; ++t) {
    const int R = kRowsPerStore * t + lane / kChunks, c = lane % kChunks;
    const u32x4 val = *reinterpret_cast<const u32x4*>(stage + R * kRowB + ((c ^ (R % kChunks)) << 4));
    if (q0 + R < Nq && (!Sh::kMaskD || c < d_chunks)) {
      u32x4* dst = reinterpret_cast<u32x4*>(ohead + (long long)(q0 + R) * row_stride + 8 * c);
      if constexpr (Sh::kMaskD)
        *dst = val;
      else
        __builtin_nontemporal_store(val, dst);
    }
  }
}

// Element strides of one (B, H, N, D) operand: batch, head, row (the last dim is contiguous).
struct Strides {
  long long b, h, n;
};

// One instance per (head dims, element type, dim masking, layout).  kDense: every operand is
// the contiguous (B, H, N, kD) layout with N_q = N_k, so row strides are compile-time and the
// stride arguments are not read.
//
// Argument order: the device pass preloads the first 14 argument dwords into SGPRs at wave
// launch (-amdgpu-kernarg-preload-count; s[0:1] hold the argument segment's address).
// Everything a dense workgroup needs before its first loads (Q, K, V, the sizes, the causal
// flag) and O and the scale sit there, so it issues its loads without a scalar load from the
// argument segment first (an L2 round trip on a CU's first workgroup: 0.3 us of a config-1
// launch).  The LSE pointer, H, D and the strides follow; the strided instances load them.
template <class Sh, bool kDense>
__global__ __launch_bounds__(kThreads, Sh::kDH == 1 ? 3 : 2) void fwd_kernel(
    const void* __restrict__ Qv, const void* __restrict__ Kv, const void* __restrict__ Vv,
    void* __restrict__ Ov, int BH, int Nq, int Nk, int nQB, int causal, float scale_log2,
    float* __restrict__ LSE, int H, int D, Strides qs, Strides ks, Strides vs, Strides os) {
  typedef typename Sh::T T;
  typedef typename Elem<T>::v8 v8;
  typedef typename Elem<T>::v4 v4;
  constexpr int kSlotBytes = Sh::kDH * kHalfTileBytes;
  constexpr int kDenseRowBytes = Sh::kD * 2;
  // The V slots first, then the K slots: a ds_read reaches 64 KiB past its base register with
  // an immediate offset, and at head dim 128 (80 KiB) only the third K slot lies beyond, read by
  // 8 of a half-step's 24 reads one tile step in three (with the V ring there, half of all
  // tile steps paid an address add per V read).
  __shared__ __attribute__((aligned(1024)))
  unsigned char ring[(Sh::kVSlots + Sh::kKSlots) * kSlotBytes];
  constexpr int kK0 = Sh::kVSlots * kSlotBytes;
  const Lds lds = {{ring + kK0, ring + kK0 + kSlotBytes, ring + kK0 + (Sh::kKSlots - 1) * kSlotBytes},
                   {ring, ring + kSlotBytes}};
  const T* Q = static_cast<const T*>(Qv);
  const T* K = static_cast<const T*>(Kv);
  const T* V = static_cast<const T*>(Vv);
  T* O = static_cast<T*>(Ov);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31;
  const int h = lane >> 5;

  // Heaviest (last) query blocks first: with causal masking block qb needs qb+1 key blocks.
  // Workgroups are dealt to the 8 XCDs (one L2 each) round-robin, so when B*H is a multiple of
  // 8 every query block of a head runs on the same XCD.
  const int bid = blockIdx.x;
  const int qb = nQB - 1 - bid / BH;
  const int bh = bid % BH;

  const int bb = bh / H, hh = bh - bb * H;
  const long long dense_head = (long long)bh * Nq * Sh::kD;
  const T* Qh = kDense ? Q + dense_head : Q + bb * qs.b + hh * qs.h;
  const int q_row_bytes = kDense ? kDenseRowBytes : (int)qs.n * 2;

  StepArgs a;
  a.k_row_bytes = kDense ? kDenseRowBytes : (int)ks.n * 2;
  a.v_row_bytes = kDense ? kDenseRowBytes : (int)vs.n * 2;
  a.k_rsrc = head_desc(kDense ? K + dense_head : K + bb * ks.b + hh * ks.h, Nk, a.k_row_bytes);
  a.v_rsrc = head_desc(kDense ? V + dense_head : V + bb * vs.b + hh * vs.h, Nk, a.v_row_bytes);
  a.d_chunks = D >> 3;
  const int q0 = qb * kBlockRows + wave * kWaveRows;  // first query row of this wave
  const int qrow = q0 + r32;                          // this lane's query row
  // Causal visibility is top-left aligned: query i sees keys j <= i (and j < Nk).
  const int kv_end = causal ? min(Nk, (qb + 1) * kBlockRows) : Nk;
  a.nT = (kv_end + kTileKeys - 1) / kTileKeys;
  // 32-key halves computed by this wave: those starting at or below its first row (causal,
  // q0 is a multiple of 32) and below Nk; unmasked: strictly below its first row (causal) and
  // wholly below Nk.
  const int nHalves = (kv_end + 31) / 32;
  if (q0 >= Nq) {
    a.nAct = 0;
    a.nFull = 0;
  } else if (causal) {
    a.nAct = min(nHalves, q0 / 32 + 1);
    a.nFull = min(q0 / 32, Nk / 32);
  } else {
    a.nAct = nHalves;
    a.nFull = Nk / 32;
  }
  a.nFull = min(a.nFull, a.nAct);
  a.wave = wave;
  a.lane = lane;
  a.h = h;
  a.last_key = causal ? min(qrow, Nk - 1) : Nk - 1;
  a.scale_log2 = scale_log2;
  a.inv_scale_log2 = 1.0f / scale_log2;

  // Q first, then the prologue tiles K_0, K_1 and V_0 (step j issues K_{j+2} and V_{j+1}).
  // Head dim 64: Q as LDS transfers into this wave's stage.  Head dim 128: ordinary buffer
  // loads into the Q registers, tracked by the compiler.
  WaveState<Sh> w;
  unsigned char* qstage = nullptr;
  if constexpr (Sh::kQStage) {
    qstage = q_stage<Sh>() + wave * (kWaveRows * kKRowBytes);
    // A wave past the last query row (q0 >= Nq) computes nothing; its stage reads row Nq - 1.
    const i32x4 qd = head_desc(Qh, Nq, q_row_bytes);
    issue_q_stage<Sh>(tile_desc(qd, min(q0, Nq - 1), q_row_bytes), q_row_bytes, qstage,
                      a.d_chunks);
  } else {
    const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<T*>(Qh), (short)0, Nq * q_row_bytes, 0x00020000);
#pragma unroll
    for (int c = 0; c < 4 * Sh::kDH; ++c) {
      int off = qrow * q_row_bytes + 32 * c + 16 * h;  // dims 16c + 8h .. +7
      if (Sh::kMaskD) off = 2 * c + h < a.d_chunks ? off : kOutOfRange;
      w.qop[c] = __builtin_bit_cast(v8, __builtin_amdgcn_raw_buffer_load_b128(qr, off, 0, 0));
    }
  }
  tile_offsets<Sh>(a.k_lane, a.v_lane, a.k_row_bytes, a.v_row_bytes, wave, lane, a.d_chunks);
  issue_tile<Sh>(a.k_rsrc, a.k_row_bytes, lds.k[0], 0, wave, a.k_lane);
  if (a.nT > 1) issue_tile<Sh>(a.k_rsrc, a.k_row_bytes, lds.k[1], kTileKeys, wave, a.k_lane);
  issue_tile<Sh>(a.v_rsrc, a.v_row_bytes, lds.v[0], 0, wave, a.v_lane);
  // The LSE pointer is not among the preloaded arguments: load it while the tiles are in flight.
  if constexpr (Sh::kLse) asm volatile("" ::"s"(LSE));

  // K A-operand, d chunk c: row r32 (+32 for the second key half, an immediate), logical 16-B
  // chunk 2c + h.
#pragma unroll
  for (int c = 0; c < 4; ++c) w.koff[c] = r32 * kKRowBytes + (((2 * c + h) ^ swz_k(r32)) << 4);
  // V^T operand, d tile dt, run s of 4 keys: source lane (group g = lane/16, j = lane%16)
  // reads V[16*cc + 8s + 4(g/2) + j/4][32dt + 16(g%2) + 4(j%4) .. +3]; the cc term and the key
  // half are immediate offsets.
  {
    const int g = lane >> 4, jj = lane & 15;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int sr = 0; sr < 2; ++sr) {
        const int row = 8 * sr + 4 * (g >> 1) + (jj >> 2);
        const int d0 = 32 * dt + 16 * (g & 1) + 4 * (jj & 3);
        w.voff[dt][sr] = row * kKRowBytes + (((d0 >> 3) ^ swz_v(row)) << 4) + (d0 & 7) * 2;
      }
  }
#pragma unroll
  for (int i = 0; i < 2 * Sh::kDH; ++i)
#pragma unroll
    for (int t = 0; t < 16; ++t) w.o[i][t] = 0.f;
  w.m_run = -INFINITY;
  w.thr = -INFINITY;
  w.l_run = 0.f;
  w.l_p = 0.f;

#pragma unroll
  for (int cc = 0; cc < 2; ++cc) w.pb[cc] = __builtin_bit_cast(v8, make_uint4(0u, 0u, 0u, 0u));

  if constexpr (Sh::kQStage) {
    // Q and K_0 have landed once K_1 and V_0 (issued after them) are all that may be in flight;
    // tile step 0 waits for those.  The barrier makes every wave's share of K_0 visible.
    if (a.nT > 1)
      wait_vmcnt<Sh::kLoadsPerWave>();
    else
      wait_vmcnt<Sh::kLoadsPerWave / 2>();
    lds_barrier();
#pragma unroll
    for (int c = 0; c < 4; ++c)
      w.qop[c] = *reinterpret_cast<const v8*>(qstage + r32 * kKRowBytes +
                                              (((2 * c + h) ^ swz_k(r32)) << 4));
  } else {
    // Wait for Q here, before the loop.  The compiler does not see the LDS transfers, so it
    // places a full vmcnt(0) before this use of the Q registers; that also covers K_0, K_1 and
    // V_0 (once, in the prologue), and leaves no compiler-tracked loads whose waits could land
    // inside the loop and drain the transfers in flight there.
#pragma unroll
    for (int c = 0; c < 4 * Sh::kDH; ++c) asm volatile("" ::"v"(w.qop[c]));
    wait_vmcnt<0>();
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    lds_barrier();
  }
  if (a.nAct > 0) w.s = qk_half<Sh, 0, 0>(w, lds);

  // Steady tile steps: both half-steps full (2j + 1 < nAct).  Tile step 0's first half-step has
  // no P.V before it.
  const int nSteady = a.nAct / 2;
  int j = 0;
  if (nSteady > 0) {
    tile_step<Sh, 0, 0, true, true>(w, lds, 0, a);
    j = 1;
    for (; j + Sh::kPeriod <= nSteady; j += Sh::kPeriod) steady_period<Sh, 1>(w, lds, j, a);
    steady_rest<Sh, 1>(w, lds, j, nSteady, a);
    j = max(j, nSteady);
  }
  // Remaining tile steps (the wave's last half and P.V, then loads and barriers only).
  for (; j < a.nT; ++j) tile_step_at<Sh, false>(w, lds, j, a);
  // P.V of the last computed half when it is the second half of the last tile (V_{nT-1}
  // landed at the last step's barrier and its slot was not refilled): half-step 2nT.
  if (a.nAct == 2 * a.nT) {
    if ((a.nT - 1) % Sh::kVSlots == 0)
      pv_half<Sh, 0, 1>(w, lds);
    else
      pv_half<Sh, 1, 1>(w, lds);
  }

  // Row sums over the lane pair (both lanes of a row hold the same offset).
  const float l_o = pair_sum(w.l_p);
  const float l_all = Sh::kLse ? pair_sum(w.l_run) : 0.f;
  // The lane's row again, from the lane id (mbcnt) rather than a value kept from the prologue:
  // a register held across the loops for the epilogue only was spilled to scratch.
  int lane_e;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane_e));
  const int qrow_e = q0 + (lane_e & 31), h_e = lane_e >> 5;
  // O leaves through LDS (store_o).  Head dim 64: the wave's own Q stage, unused since the
  // prologue.  Head dim 128: a share of the K/V ring, free once every wave is past this barrier
  // (every K/V read was consumed by an MFMA, every transfer waited for).
  unsigned char* ostage;
  if constexpr (Sh::kQStage) {
    ostage = qstage;
  } else {
    lds_barrier();
    ostage = ring + wave * (kWaveRows * Sh::kD * 2);
  }
  T* ohead = kDense ? O + dense_head : O + bb * os.b + hh * os.h;
  store_o<Sh>(w, ostage, 1.0f / l_o, lane_e, ohead, kDense ? (long long)Sh::kD : os.n, q0, Nq,
              a.d_chunks);
  if (Sh::kLse && LSE != nullptr && h_e == 0 && qrow_e < Nq)
    LSE[(size_t)bh * Nq + qrow_e] = (w.m_run + __builtin_amdgcn_logf(l_all)) * kLn2;
}

// ---------------------------------------------------------------------------------------
// Small grids: split-key workgroups (fwd_split_kernel).
//
// When B * H * ceil(N_q / 128) workgroups of fwd_kernel leave most CUs idle, a launch takes as
// long as its longest wave's chain of half-steps (4qb + 4 for query block qb), not its work.
// Then each workgroup takes one 32-row query block, and its 4 waves split the block's 32-key
// halves (wave w: halves w, w + 4, w + 8, ...): every wave runs its own online softmax over the
// same 32 rows, with its own 2-slot ring of K and V halves in LDS, so no wave waits for another
// until the merge.  The merge goes through LDS with the log-sum-exp rule over the 4 partial
// states (offset m_w, rounded-probability sum lp_w, fp32 sum l_w, unnormalised O_w):
//   M = max_w m_w,  a_w = 2^(m_w - M),  O = sum_w a_w O_w / sum_w a_w lp_w,
//   LSE = (M + log2 sum_w a_w l_w) ln 2.
// A wave with no half contributes m_w = -inf (a_w = 0).  The half-step is the tail path of
// fwd_kernel (qk_half, mask_half, move_offset, exp_half, pv_half), unpipelined: at this size
// the time is latency, and each wave has at most ceil(nH / 4) halves.  A wave with exactly two
// (both loaded by the prologue) computes them together (split_pair): at B1 H12 N256 that took
// the launch from 5.06 to 4.19 us.
constexpr int kHalfBytes = 32 * kKRowBytes;  // one 32-key half of K or V, one dim half: 4 KiB

template <class Sh>
struct SplitLayout {
  // Waves per workgroup.  8 at head dim 64 (one half per wave at N = 256) measured no faster
  // at B1 H12 N256 and slower from N = 1024 on.
  static constexpr int kWaves = 4;
  static constexpr int kSlotBytes = 2 * Sh::kDH * kHalfBytes;  // a K half, then a V half
  static constexpr int kWaveBytes = 2 * kSlotBytes;             // the wave's 2-slot ring
  static constexpr int kRingBytes = kWaves * kWaveBytes;
  static constexpr int kQBytes = kWaveRows * Sh::kD * 2;        // the block's 32 Q rows
  static constexpr int kOPartBytes = kWaveRows * Sh::kD * 4;    // one wave's O partial, fp32
  static_assert(kWaves * kOPartBytes <= kRingBytes, "the O partials fit in the rings");
  static constexpr int kLoadsPerHalf = 8 * Sh::kDH;             // 1-KiB transfers, K and V
  static constexpr int kRowsPerWave = kWaveRows / kWaves;       // rows each wave merges
};

// Rows r0 .. r0 + 7 of one 32-row half (dim half dh) from the buffer at `desc` (rows row_bytes
// apart) into LDS at dst + 128 * r0: lane i fills physical chunk i % 8 of row r0 + i / 8 with
// the logical chunk the swizzle maps there (K swizzle for K and Q, V swizzle for V).
template <class Sh, bool kVSwz>
__device__ __forceinline__ void issue_rows8(i32x4 desc, int row_bytes, unsigned char* dst, int r0,
                                            int dh, int lane, int d_chunks) {
  const int row = r0 + (lane >> 3);
  const int lc = 8 * dh + ((lane & 7) ^ (kVSwz ? swz_v(row) : swz_k(row)));
  int off = row * row_bytes + (lc << 4);
  if (Sh::kMaskD) off = lc < d_chunks ? off : kOutOfRange;
  lds_transfer(desc, lds_addr(dst + r0 * kKRowBytes), off);
}

// Half u of K and V (32 rows each, every dim half) into ring slot `slot` of this wave.
template <class Sh>
__device__ __forceinline__ void issue_split_half(const StepArgs& a, unsigned char* slot, int u) {
  const i32x4 kd = tile_desc(a.k_rsrc, 32 * u, a.k_row_bytes);
  const i32x4 vd = tile_desc(a.v_rsrc, 32 * u, a.v_row_bytes);
  unsigned char* vslot = slot + Sh::kDH * kHalfBytes;
#pragma unroll
  for (int dh = 0; dh < Sh::kDH; ++dh)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      issue_rows8<Sh, false>(kd, a.k_row_bytes, slot + dh * kHalfBytes, 8 * t, dh, a.lane, a.d_chunks);
      issue_rows8<Sh, true>(vd, a.v_row_bytes, vslot + dh * kHalfBytes, 8 * t, dh, a.lane, a.d_chunks);
    }
}

// One half u from ring slot kSlot: S, mask (diagonal or last partial half), offset check, P and
// its sums, O += V P.
template <class Sh, int kSlot>
__device__ __forceinline__ void split_half(WaveState<Sh>& w, const Lds& lds, int u, const StepArgs& a) {
  w.s = qk_half<Sh, kSlot, 0, kHalfBytes>(w, lds);
  if (u >= a.nFull) mask_half(w, a.last_key - u * 32 - 4 * a.h);
  move_offset(w, lane_max(w), a.scale_log2, a.inv_scale_log2);
  exp_half(w, a.scale_log2);
  pv_half<Sh, kSlot, 0, kHalfBytes>(w, lds);
}

// Halves u0 (ring slot 0) and u1 (slot 1) together: two independent S chains, one offset check
// over both (every P of both halves is then within the margin), then P and O += V P for each.
// For a wave with exactly two halves, the common case of the latency-bound grids this kernel
// runs, this is a shorter dependency chain than two split_half calls.
template <class Sh>
__device__ __forceinline__ void split_pair(WaveState<Sh>& w, const Lds& lds, int u0, int u1,
                                           const StepArgs& a) {
  const f32x16 s0 = qk_half<Sh, 0, 0, kHalfBytes>(w, lds);
  w.s = qk_half<Sh, 1, 0, kHalfBytes>(w, lds);
  if (u1 >= a.nFull) mask_half(w, a.last_key - u1 * 32 - 4 * a.h);
  const float mx1 = lane_max(w);
  const f32x16 s1 = w.s;
  w.s = s0;
  if (u0 >= a.nFull) mask_half(w, a.last_key - u0 * 32 - 4 * a.h);
  move_offset(w, fmaxf(lane_max(w), mx1), a.scale_log2, a.inv_scale_log2);
  exp_half(w, a.scale_log2);
  pv_half<Sh, 0, 0, kHalfBytes>(w, lds);
  w.s = s1;
  exp_half(w, a.scale_log2);
  pv_half<Sh, 1, 0, kHalfBytes>(w, lds);
}

// Arguments in fwd_kernel's order (the preloaded dwords first).  kDense as for fwd_kernel; the
// dense instances are what makes a small contiguous launch start without a scalar load (B1 H12
// N256: 4.10 -> 3.76 us).
template <class Sh, bool kDense>
__global__ __launch_bounds__(SplitLayout<Sh>::kWaves * 64, 1) void fwd_split_kernel(
    const void* __restrict__ Qv, const void* __restrict__ Kv, const void* __restrict__ Vv,
    void* __restrict__ Ov, int BH, int Nq, int Nk, int nRB, int causal, float scale_log2,
    float* __restrict__ LSE, int H, int D, Strides qs, Strides ks, Strides vs, Strides os) {
  typedef typename Sh::T T;
  typedef typename Elem<T>::v8 v8;
  typedef SplitLayout<Sh> L;
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  __shared__ __attribute__((aligned(1024))) unsigned char ring[L::kRingBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char qst[L::kQBytes];
  __shared__ float stats[L::kWaves][3][kWaveRows];  // m, lp, l per wave and row

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31;
  const int h = lane >> 5;
  // Heaviest (last) query blocks first.
  const int bid = blockIdx.x;
  const int rb = nRB - 1 - bid / BH;
  const int bh = bid % BH;
  const int bb = kDense ? 0 : bh / H, hh = kDense ? 0 : bh - bb * H;
  const long long dense_head = (long long)bh * Nq * Sh::kD;
  const T* Q = static_cast<const T*>(Qv) + (kDense ? dense_head : bb * qs.b + hh * qs.h);
  const T* K = static_cast<const T*>(Kv) + (kDense ? dense_head : bb * ks.b + hh * ks.h);
  const T* V = static_cast<const T*>(Vv) + (kDense ? dense_head : bb * vs.b + hh * vs.h);
  const int q_row_bytes = kDense ? Sh::kD * 2 : (int)qs.n * 2;
  const int q0 = rb * kWaveRows;
  const int qrow = q0 + r32;

  StepArgs a;
  a.k_row_bytes = kDense ? Sh::kD * 2 : (int)ks.n * 2;
  a.v_row_bytes = kDense ? Sh::kD * 2 : (int)vs.n * 2;
  a.k_rsrc = head_desc(K, Nk, a.k_row_bytes);
  a.v_rsrc = head_desc(V, Nk, a.v_row_bytes);
  a.d_chunks = D >> 3;
  // Halves of the block: those starting at or below its last row (causal, top-left aligned) and
  // below Nk; unmasked: wholly below its first row (causal) and wholly below Nk.
  const int kv_end = causal ? min(Nk, q0 + kWaveRows) : Nk;
  const int nH = (kv_end + 31) / 32;
  a.nFull = causal ? min(q0 / 32, Nk / 32) : Nk / 32;
  a.nAct = wave < nH ? (nH - 1 - wave) / L::kWaves + 1 : 0;  // this wave's halves
  a.nT = 0;
  a.wave = wave;
  a.lane = lane;
  a.h = h;
  a.last_key = causal ? min(qrow, Nk - 1) : Nk - 1;
  a.scale_log2 = scale_log2;
  a.inv_scale_log2 = 1.0f / scale_log2;

  unsigned char* wring = ring + wave * L::kWaveBytes;
  const Lds lds = {{wring, wring + L::kSlotBytes, nullptr},
                   {wring + Sh::kDH * kHalfBytes, wring + L::kSlotBytes + Sh::kDH * kHalfBytes}};

  // This wave's quarter of the Q block (rows 8w .. 8w + 7 of each dim half), then its first two
  // halves.  Rows past N_q read zero.
  if (wave < kWaveRows / 8) {
    const i32x4 qd = tile_desc(head_desc(Q, Nq, q_row_bytes), q0, q_row_bytes);
#pragma unroll
    for (int dh = 0; dh < Sh::kDH; ++dh)
      issue_rows8<Sh, false>(qd, q_row_bytes, qst + dh * kHalfBytes, 8 * wave, dh, lane, a.d_chunks);
  }
  if (a.nAct > 0) issue_split_half<Sh>(a, wring, wave);
  if (a.nAct > 1) issue_split_half<Sh>(a, wring + L::kSlotBytes, wave + L::kWaves);
  // The LSE pointer is not preloaded: load it while the halves are in flight, not at the store.
  if constexpr (Sh::kLse) asm volatile("" ::"s"(LSE));

  WaveState<Sh> w;
#pragma unroll
  for (int c = 0; c < 4; ++c) w.koff[c] = r32 * kKRowBytes + (((2 * c + h) ^ swz_k(r32)) << 4);
  {
    const int g = lane >> 4, jj = lane & 15;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int sr = 0; sr < 2; ++sr) {
        const int row = 8 * sr + 4 * (g >> 1) + (jj >> 2);
        const int d0 = 32 * dt + 16 * (g & 1) + 4 * (jj & 3);
        w.voff[dt][sr] = row * kKRowBytes + (((d0 >> 3) ^ swz_v(row)) << 4) + (d0 & 7) * 2;
      }
  }
#pragma unroll
  for (int i = 0; i < 2 * Sh::kDH; ++i)
#pragma unroll
    for (int t = 0; t < 16; ++t) w.o[i][t] = 0.f;
  w.m_run = -INFINITY;
  w.thr = -INFINITY;
  w.l_run = 0.f;
  w.l_p = 0.f;

  // Q has landed once only the half transfers (issued after it) may be in flight; the barrier
  // makes every wave's quarter visible.
  if (a.nAct > 1)
    wait_vmcnt<2 * L::kLoadsPerHalf>();
  else if (a.nAct == 1)
    wait_vmcnt<L::kLoadsPerHalf>();
  else
    wait_vmcnt<0>();
  lds_barrier();
#pragma unroll
  for (int dh = 0; dh < Sh::kDH; ++dh)
#pragma unroll
    for (int c = 0; c < 4; ++c)
      w.qop[4 * dh + c] = *reinterpret_cast<const v8*>(qst + dh * kHalfBytes + r32 * kKRowBytes +
                                                        (((2 * c + h) ^ swz_k(r32)) << 4));

  if (a.nAct == 2) {
    // Both halves were issued by the prologue.
    wait_vmcnt<0>();
    split_pair<Sh>(w, lds, wave, wave + L::kWaves, a);
  } else {
  for (int i = 0; i < a.nAct; ++i) {
    const int u = wave + L::kWaves * i;
    if (i + 1 < a.nAct)
      wait_vmcnt<L::kLoadsPerHalf>();
    else
      wait_vmcnt<0>();
    if (i & 1)
      split_half<Sh, 1>(w, lds, u, a);
    else
      split_half<Sh, 0>(w, lds, u, a);
    if (i + 2 < a.nAct) {
      // The slot's LDS reads are complete before the transfers into it are issued.
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      issue_split_half<Sh>(a, wring + (i & 1) * L::kSlotBytes, u + 2 * L::kWaves);
    }
  }
  }

  // Merge.  Each wave publishes its row statistics and its unnormalised O rows (fp32, row-major,
  // 16-B chunk c of row r at physical chunk c ^ (r % (kD/4))) over its own ring, which only it
  // used: its transfers were all waited for, and its LDS accesses complete in order, so its K/V
  // reads come before these writes.  One barrier then publishes every wave's rows.
  const float lp = pair_sum(w.l_p);
  const float lr = Sh::kLse ? pair_sum(w.l_run) : 0.f;
  int lane_e;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane_e));
  const int r_e = lane_e & 31, h_e = lane_e >> 5;
  constexpr int kC4 = Sh::kD / 4;   // 16-B fp32 chunks per O row
  constexpr int kRowB = Sh::kD * 4;
  static_assert(L::kOPartBytes <= L::kWaveBytes, "a wave's O partial fits in its ring");
  unsigned char* opart = wring;
#pragma unroll
  for (int i = 0; i < 2 * Sh::kDH; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      // Register 4g + e of tile i holds dim 32i + 8g + 4h + e: fp32 chunk 8i + 2g + h.
      const f32x4 x = {w.o[i][4 * g], w.o[i][4 * g + 1], w.o[i][4 * g + 2], w.o[i][4 * g + 3]};
      const int c = 8 * i + 2 * g + h_e;
      *reinterpret_cast<f32x4*>(opart + r_e * kRowB + ((c ^ (r_e % kC4)) << 4)) = x;
    }
  if (h_e == 0) {
    stats[wave][0][r_e] = w.m_run;
    stats[wave][1][r_e] = lp;
    stats[wave][2][r_e] = lr;
  }
  lds_write_barrier();
  // Wave w combines rows w * kRowsPerWave .. +kRowsPerWave - 1: item -> (row, 8 head dims),
  // kD/8 items per row, so each lane stores 16 B and kD/8 lanes a whole row (non-temporal, as
  // in store_o).
  constexpr int kC8 = Sh::kD / 8;
  constexpr int kItems = L::kRowsPerWave * kC8;
  T* O = static_cast<T*>(Ov) + (kDense ? dense_head : bb * os.b + hh * os.h);
  const long long o_rs = kDense ? (long long)Sh::kD : os.n;
#pragma unroll
  for (int pass = 0; pass < (kItems + 63) / 64; ++pass) {
    const int item = 64 * pass + lane_e;
    if (kItems % 64 != 0 && item >= kItems) break;
    const int R = L::kRowsPerWave * wave + item / kC8, c8 = item % kC8;
    float M = -INFINITY;
#pragma unroll
    for (int v = 0; v < L::kWaves; ++v) M = fmaxf(M, stats[v][0][R]);
    float lsum = 0.f, lrun = 0.f;
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int v = 0; v < L::kWaves; ++v) {
      const float av = __builtin_amdgcn_exp2f(stats[v][0][R] - M);
      lsum = fmaf(av, stats[v][1][R], lsum);
      if constexpr (Sh::kLse) lrun = fmaf(av, stats[v][2][R], lrun);
      const unsigned char* src = ring + v * L::kWaveBytes + R * kRowB;
      const f32x4 x0 = *reinterpret_cast<const f32x4*>(src + (((2 * c8) ^ (R % kC4)) << 4));
      const f32x4 x1 = *reinterpret_cast<const f32x4*>(src + (((2 * c8 + 1) ^ (R % kC4)) << 4));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc0[e] = fmaf(av, x0[e], acc0[e]);
        acc1[e] = fmaf(av, x1[e], acc1[e]);
      }
    }
    const float inv = 1.0f / lsum;
    typename Elem<T>::v8 ov;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      ov[e] = (T)(acc0[e] * inv);
      ov[4 + e] = (T)(acc1[e] * inv);
    }
    const int qr = q0 + R;
    if (qr < Nq && (!Sh::kMaskD || c8 < a.d_chunks)) {
      u32x4* dst = reinterpret_cast<u32x4*>(O + (long long)qr * o_rs + 8 * c8);
      if constexpr (Sh::kMaskD)
        *dst = __builtin_bit_cast(u32x4, ov);
      else
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4, ov), dst);
    }
    if (Sh::kLse && LSE != nullptr && c8 == 0 && qr < Nq)
      LSE[(size_t)bh * Nq + qr] = (M + __builtin_amdgcn_logf(lrun)) * kLn2;
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

// Element strides of one operand as the kernel uses them.  A null `st` is the contiguous
// (B, H, N, D) layout.  The stride of a dimension of size 1 is never used (it may hold
// anything, as in torch), so it is replaced by 0 (b, h) or D (n).
static Strides operand_strides(const int64_t* st, int B, int H, int N, int D) {
  Strides s;
  s.b = B == 1 ? 0 : st ? st[0] : (long long)H * N * D;
  s.h = H == 1 ? 0 : st ? st[1] : (long long)N * D;
  s.n = N == 1 ? D : st ? st[2] : D;
  return s;
}

// Stride rules (elements): the last dimension is dense (stride 1); the row stride is at least
// D, so rows of one head do not overlap and row N starts where a buffer descriptor over N
// rows ends; every stride is a non-negative multiple of 8, so every row start keeps the
// 16-byte alignment of the base pointer; the largest per-head buffer offset,
// (N + 128) rows * row stride * 2 bytes + the row's 2 * 128 bytes, fits the 32-bit offset of
// a buffer access.
static int check_strides(const int64_t* st, int B, int H, int N, int D) {
  const Strides s = operand_strides(st, B, H, N, D);
  if (st != nullptr) {
    if (st[3] != 1) return TFGFA_ERR_STRIDE;
    if (s.b < 0 || s.h < 0 || s.n < D) return TFGFA_ERR_STRIDE;
    if ((s.b | s.h | s.n) & 7) return TFGFA_ERR_STRIDE;
  }
  if (s.n > INT32_MAX / 2 || ((long long)N + kBlockRows) * s.n * 2 + 2 * kMaxD > INT32_MAX)
    return TFGFA_ERR_TOO_LARGE;
  return TFGFA_OK;
}

// O must not write one element twice: with its dimensions of size > 1 sorted by stride, each
// stride must exceed the largest offset reachable through the smaller ones (a sufficient
// condition for distinct offsets; every layout torch makes by viewing a buffer meets it).
static bool overlaps(const int64_t* st, int B, int H, int N, int D) {
  if (st == nullptr) return false;
  const Strides s = operand_strides(st, B, H, N, D);
  long long stride[3] = {s.b, s.h, s.n};
  long long size[3] = {B, H, N};
  for (int i = 0; i < 3; ++i)  // insertion sort by stride, 3 elements
    for (int j = i; j > 0 && stride[j] < stride[j - 1]; --j) {
      const long long ts = stride[j], tz = size[j];
      stride[j] = stride[j - 1];
      size[j] = size[j - 1];
      stride[j - 1] = ts;
      size[j - 1] = tz;
    }
  long long reach = D - 1;  // the dense last dimension
  for (int i = 0; i < 3; ++i) {
    if (size[i] == 1) continue;
    if (stride[i] <= reach) return true;
    reach += (size[i] - 1) * stride[i];
  }
  return false;
}

// Argument checks, in this order: sizes, flags and strides first, then - only for a non-empty
// problem - pointers.  An empty tensor may legitimately have a null data pointer
// (torch gives numel()==0 tensors address 0), so B, H or N_q == 0 succeeds with no launch.
static int validate(const void* q, const void* k, const void* v, const void* o, const float* lse,
                    int B, int H, int Nq, int Nk, int D, int dtype, float scale, int causal,
                    const int64_t* const* st) {
  if (B < 0 || H < 0 || Nq < 0 || Nk < 0) return TFGFA_ERR_BAD_SHAPE;
  if (D < 8 || D > kMaxD || (D & 7)) return TFGFA_ERR_HEAD_DIM;
  if (dtype != TFGFA_DTYPE_BF16 && dtype != TFGFA_DTYPE_F16) return TFGFA_ERR_DTYPE;
  if (!(scale > 0.f) || !isfinite(scale)) return TFGFA_ERR_SCALE;
  if (causal != 0 && causal != 1) return TFGFA_ERR_CAUSAL_FLAG;
  if (B == 0 || H == 0 || Nq == 0) return TFGFA_OK;
  if (Nk == 0) return TFGFA_ERR_BAD_SHAPE;  // every query row needs a key
  const long long bh = (long long)B * H;
  const long long nqb = ((long long)Nq + kBlockRows - 1) / kBlockRows;
  if (bh > INT32_MAX || bh * nqb > INT32_MAX) return TFGFA_ERR_TOO_LARGE;
  const int rows[4] = {Nq, Nk, Nk, Nq};
  for (int i = 0; i < 4; ++i) {
    const int sst = check_strides(st[i], B, H, rows[i], D);
    if (sst != TFGFA_OK) return sst;
  }
  if (overlaps(st[3], B, H, Nq, D)) return TFGFA_ERR_STRIDE;
  if (q == nullptr || k == nullptr || v == nullptr || o == nullptr) return TFGFA_ERR_NULL_POINTER;
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)o) & 15u) return TFGFA_ERR_ALIGNMENT;
  if (((uintptr_t)lse) & 3u) return TFGFA_ERR_ALIGNMENT;
  return TFGFA_OK;
}

// fwd_kernel's grid of 128-row query blocks is at most one workgroup per CU: the split-key
// kernel runs the launch instead (a 4x larger grid, a longest wave chain about 4x shorter).
// Measured crossover (bf16, head dims 64 and 128): faster at every grid up to the CU count
// (B1 H12 N256 6.66 -> 5.07 us, B1 H16 N1024 15.9 -> 10.1 us, B1 H16 N2048 27.9 -> 24.6 us),
// slower from twice that (B2 H32 N1024 17.5 -> 27.9 us).  The choice depends on the sizes only,
// never on strides or outputs, so every instance of one problem takes the same arithmetic.
static bool use_split_grid(long long blocks, int cu_count) { return blocks <= cu_count; }

struct LaunchArgs {
  const void *q, *k, *v;
  void* o;
  float* lse;
  int H, BH, Nq, Nk, D, nQB;
  float scale_log2;
  int causal;
  Strides qs, ks, vs, os;
};

template <class Sh, bool kDense>
static void launch_instance(const LaunchArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((fwd_kernel<Sh, kDense>), dim3(a.BH * a.nQB), dim3(kThreads), 0, stream, a.q,
                     a.k, a.v, a.o, a.BH, a.Nq, a.Nk, a.nQB, a.causal, a.scale_log2, a.lse, a.H,
                     a.D, a.qs, a.ks, a.vs, a.os);
}

template <class Sh, bool kDense = false>
static void launch_split_instance(const LaunchArgs& a, hipStream_t stream) {
  const int nRB = (a.Nq + kWaveRows - 1) / kWaveRows;
  hipLaunchKernelGGL((fwd_split_kernel<Sh, kDense>), dim3(a.BH * nRB),
                     dim3(SplitLayout<Sh>::kWaves * 64), 0, stream, a.q, a.k, a.v, a.o, a.BH,
                     a.Nq, a.Nk, nRB, a.causal, a.scale_log2, a.lse, a.H, a.D, a.qs, a.ks, a.vs,
                     a.os);
}

template <int kD, typename T>
static void launch_dims(const LaunchArgs& a, bool dense, bool split, hipStream_t stream) {
  if (split) {
    if constexpr (kD == 64 && std::is_same<T, __bf16>::value) {
      if (dense && a.D == kD) {  // the reference's layout: no stride arguments to load
        if (a.lse != nullptr)
          launch_split_instance<Shape<kD, T, false>, true>(a, stream);
        else
          launch_split_instance<Shape<kD, T, false, false>, true>(a, stream);
        return;
      }
    }
    if (a.D != kD)
      launch_split_instance<Shape<kD, T, true>>(a, stream);
    else if (a.lse != nullptr)
      launch_split_instance<Shape<kD, T, false>>(a, stream);
    else
      launch_split_instance<Shape<kD, T, false, false>>(a, stream);
    return;
  }
  if (a.D != kD) {
    launch_instance<Shape<kD, T, true>, false>(a, stream);
    return;
  }
  if constexpr (kD == 64 && std::is_same<T, __bf16>::value) {
    if (dense) {  // the GPT-2 layout
      if (a.lse != nullptr)
        launch_instance<Shape<kD, T, false>, true>(a, stream);
      else
        launch_instance<Shape<kD, T, false, false>, true>(a, stream);
      return;
    }
  }
  if (a.lse != nullptr)
    launch_instance<Shape<kD, T, false>, false>(a, stream);
  else
    launch_instance<Shape<kD, T, false, false>, false>(a, stream);
}

static int launch(const void* q, const void* k, const void* v, void* o, float* lse, int B, int H,
                  int Nq, int Nk, int D, int dtype, float softmax_scale, int causal,
                  void* hip_stream, const int64_t* const* st) {
  const int vst = validate(q, k, v, o, lse, B, H, Nq, Nk, D, dtype, softmax_scale, causal, st);
  if (vst != TFGFA_OK) return vst;
  if (B == 0 || H == 0 || Nq == 0) return TFGFA_OK;

  LaunchArgs a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.lse = lse;
  a.H = H;
  a.BH = B * H;
  a.Nq = Nq;
  a.Nk = Nk;
  a.D = D;
  a.nQB = (Nq + kBlockRows - 1) / kBlockRows;
  a.scale_log2 = softmax_scale * kLog2e;
  a.causal = causal;
  a.qs = operand_strides(st[0], B, H, Nq, D);
  a.ks = operand_strides(st[1], B, H, Nk, D);
  a.vs = operand_strides(st[2], B, H, Nk, D);
  a.os = operand_strides(st[3], B, H, Nq, D);
  const Strides dq = operand_strides(nullptr, B, H, Nq, D);
  auto same = [](const Strides& x, const Strides& y) {
    return x.b == y.b && x.h == y.h && x.n == y.n;
  };
  const bool dense = Nq == Nk && same(a.qs, dq) && same(a.ks, dq) && same(a.vs, dq) && same(a.os, dq);
  int cu_count = 0;
  const int ist = tfgfa_device_info(&cu_count, nullptr, nullptr, 0);
  if (ist != TFGFA_OK) return ist;
  const bool split = use_split_grid((long long)a.BH * a.nQB, cu_count);
  const hipStream_t stream = (hipStream_t)hip_stream;
  if (dtype == TFGFA_DTYPE_BF16) {
    if (D <= 64)
      launch_dims<64, __bf16>(a, dense, split, stream);
    else
      launch_dims<128, __bf16>(a, dense, split, stream);
  } else {
    if (D <= 64)
      launch_dims<64, _Float16>(a, dense, split, stream);
    else
      launch_dims<128, _Float16>(a, dense, split, stream);
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? TFGFA_OK : -(int)e;
}

}  // namespace tfgfa

extern "C" int tfgfa_fwd(const void* q, const int64_t* q_strides, const void* k,
                         const int64_t* k_strides, const void* v, const int64_t* v_strides,
                         void* o, const int64_t* o_strides, float* lse, int B, int H, int N_q,
                         int N_k, int D, int dtype, float softmax_scale, int causal,
                         void* hip_stream) {
  const int64_t* const st[4] = {q_strides, k_strides, v_strides, o_strides};
  return tfgfa::launch(q, k, v, o, lse, B, H, N_q, N_k, D, dtype, softmax_scale, causal,
                       hip_stream, st);
}

extern "C" int tfgfa_fwd_bf16(const void* q, const void* k, const void* v, void* o, float* lse,
                              int B, int H, int N, int D, float softmax_scale, int causal,
                              void* hip_stream) {
  const int64_t* const contiguous[4] = {nullptr, nullptr, nullptr, nullptr};
  return tfgfa::launch(q, k, v, o, lse, B, H, N, N, D, TFGFA_DTYPE_BF16, softmax_scale, causal,
                       hip_stream, contiguous);
}

extern "C" int tfgfa_fwd_bf16_strided(const void* q, const int64_t* q_strides, const void* k,
                                      const int64_t* k_strides, const void* v,
                                      const int64_t* v_strides, void* o,
                                      const int64_t* o_strides, float* lse, int B, int H, int N,
                                      int D, float softmax_scale, int causal, void* hip_stream) {
  const int64_t* const st[4] = {q_strides, k_strides, v_strides, o_strides};
  return tfgfa::launch(q, k, v, o, lse, B, H, N, N, D, TFGFA_DTYPE_BF16, softmax_scale, causal,
                       hip_stream, st);
}

extern "C" const char* tfgfa_strerror(int status) {
  switch (status) {
    case TFGFA_OK: return "success";
    case TFGFA_ERR_NULL_POINTER: return "null tensor pointer (q, k, v and o are required)";
    case TFGFA_ERR_BAD_SHAPE:
      return "negative batch, head or sequence size, or no keys for a non-empty query";
    case TFGFA_ERR_HEAD_DIM: return "unsupported head dimension (a multiple of 8 up to 128)";
    case TFGFA_ERR_DTYPE: return "unsupported dtype (TFGFA_DTYPE_BF16 or TFGFA_DTYPE_F16)";
    case TFGFA_ERR_SCALE: return "softmax_scale must be finite and > 0";
    case TFGFA_ERR_CAUSAL_FLAG: return "causal flag must be 0 or 1";
    case TFGFA_ERR_TOO_LARGE: return "problem exceeds the launch limits (B*H*ceil(N/128) < 2^31)";
    case TFGFA_ERR_ALIGNMENT: return "misaligned pointer (q/k/v/o need 16 B, lse 4 B)";
    case TFGFA_ERR_CACHE: return "k_new/v_new (cache append) need cache_seqlens";
    case TFGFA_ERR_SCRATCH:
      return "reserved status (decode scratch): not returned by this library";
    case TFGFA_ERR_STRIDE:
      return "unsupported strides (last dim 1; b, h, n non-negative multiples of 8; n >= head dim; "
             "o without overlapping elements)";
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
