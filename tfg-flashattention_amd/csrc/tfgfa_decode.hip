// tfgfa_decode.hip - one decode step of attention over a KV cache, MI355X (gfx950), bf16 or
// fp16, head dim a multiple of 8 up to 128.
//
// What it replaces: the reference's generate() has no KV cache; every new token re-runs the
// whole prefix through the model, i.e. a full causal forward of which only the last query row
// is kept (src/py/model_inference.py:199-228, timed at :444-457).  The last row of that causal
// forward is exactly attention of one query over all cached keys:
//     o = softmax_j(scale * q . k_j) v_j,  j < L,   lse = log sum_j exp(scale * q . k_j)
// (the same math as model_inference.py:68-75 restricted to row L-1).  This file computes that
// row directly from a cache, optionally appending the new token's k/v first.
//
// Bound: HBM.  Every cached K and V byte is read once (4D bytes per key per head) and the
// arithmetic is 2D MACs per key, about 0.5 FLOP/B, so the MFMA units have nothing to do:
// scores and the P.V update are VALU v_dot2_f32_{bf16,f16} on the values as loaded (two MACs
// per instruction, fp32 accumulate), which keeps the VALU time per byte below the HBM time.
//
// Work decomposition (split over the cache sequence)
//   grid = B * H * S workgroups of kW waves; workgroup (bh, s) covers keys [s*C, s*C + C) of
//   head bh.  S = 1 (8-wave workgroups, one per head) while B*H exceeds half the CUs; at or
//   below that the host splits each head over 4-wave workgroups that fill one round of
//   workgroup slots (choose_split).  Inside a workgroup, wave w takes 32-key blocks w, w+kW,
//   w+2kW, ... of the chunk.
//   Lane l of a wave handles keys (block + l/4) and (block + l/4 + 16) and, for each 32-dim
//   piece p of the row, head dims 32p + 8c .. 32p + 8c + 7 (c = l%4): one buffer_load_dwordx4
//   per piece per key row per lane, so a wave instruction reads 16 rows x 64 contiguous bytes.
//   Pieces at or past the head dim load from an out-of-range offset (zeros, no memory access)
//   and are never stored.  The next block's K and V loads are issued before the current
//   block is computed.
//   Each quad of lanes (one key column of the wave) runs its own online softmax over its
//   keys, so the only cross-lane step per block is the 2-step DPP sum of a dot product within
//   the quad; the 16 kW streams of a workgroup (in LDS) and, when S > 1, the workgroups are
//   merged once at the end with the log-sum-exp rule
//   o = sum_i 2^(m_i - M) o_i / sum_i 2^(m_i - M) l_i.
//   S = 1: the workgroup writes O and LSE itself.
//   S > 1, one kernel: each workgroup writes its normalised partial (o_s[D], log2-domain
//   lse_s) to the workspace and counts its arrival on the head's arrival word; the workgroup
//   that arrives last merges the head's S partials and writes O and LSE (arrival protocol
//   below).  A second, merging kernel would cost a launch and a drain per step (measured
//   1.6 us for an empty kernel between graph-replayed kernels).
//
// Arrival protocol (S > 1).  The workspace starts with one 64-bit word per head, 128 bytes
// apart (heads do not share a cache line: atomics on one line serialise), holding
// tag << 16 | count.  The host draws a random nonzero 48-bit tag per call.
//   start: wave 0 reads the word (before its first cache loads); when the tag differs (an idle
//     word, 0, or memory never used as a workspace), lane 0 swaps in (tag, 0) with one
//     compare-and-swap whose result is not needed: it fails only when another workgroup of
//     the call already installed the tag.  The latency hides behind the cache loads.
//   end: the partial is written with agent-coherent stores and waited for (s_waitcnt vmcnt(0):
//     the stores have reached the device coherence point), then the count is incremented with
//     one relaxed agent-scope atomic; the workgroup that reads count S - 1 resets the word to
//     0 and reads the partials with agent-coherent loads.  Stores that bypass the
//     non-coherent per-XCD L2 plus the wait stand in for a release fence, whose L2 writeback
//     costs ~35 ns per workgroup serialised (measured: 30.7 us against 10.9 us per step at
//     1 x 16 heads x 8192 rows).
//   Every completed call leaves the words at 0, so the workspace needs no initialisation:
//   garbage breaks the count only if its upper 48 bits equal this call's random tag.  Graph
//   replays reuse the captured tag, each starting from the 0 the previous replay left.
//
// Cache append: with k_new/v_new given, key L_b = cache_seqlens[b] is the new token: the
// workgroup whose chunk holds it stores k_new/v_new into cache row L_b and folds the values
// from the inputs into one softmax stream (no workgroup reads that row from the cache), and
// attention covers L_b + 1 keys.
// Loads of cache rows at or past L_b return zero (buffer range check, num_records = L_b rows).
// The one exception is each wave's first block, issued before L_b arrives from memory: it
// reads within the cache allocation (N_max rows), and its rows at or past L_b are zeroed in
// registers before use.  No value of a row at or past L_b reaches the result.
//
// Invalid lengths (L_b < 0 or L_b + append > N_max) cannot be rejected before launch (they
// live in device memory): for such a batch row the kernel writes NaN to O and LSE, attends no
// key and appends nothing.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <mutex>

#include "tfgfa.h"

namespace tfgfa_dec {

constexpr int kD = 64;                         // head dim of tfgfa_decode_bf16
constexpr int kMaxD = 128;                     // largest head dim of tfgfa_decode
constexpr int kWavesWhole = 8;                 // waves per workgroup, one workgroup per head
constexpr int kWavesSplit = 4;                 // waves per workgroup of a split head
constexpr int kKeysPerLane = 2;                // keys per lane per block (rows 16 apart)
static_assert(kKeysPerLane % 2 == 0, "P.V pairs keys");
constexpr int kWaveKeys = 16 * kKeysPerLane;   // keys per wave per block
constexpr int kBlockKeys = kWavesWhole * kWaveKeys;       // chunk granule, one workgroup per head
constexpr int kSplitBlockKeys = kWavesSplit * kWaveKeys;  // chunk granule of a split head
constexpr int kGroups = 16;                    // key columns per wave (4 lanes each)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kWorkspaceRows = 128;            // cache rows per split counted by the workspace
static_assert(kSplitBlockKeys % kWorkspaceRows == 0, "splits must not outnumber workspace slots");
constexpr int kArriveStride = 128;             // bytes between the arrival words of two heads
constexpr int kTagShift = 16;                  // arrival word: tag << 16 | count (count < 2^16)
// A buffer offset past any num_records this file builds (those stay below 2^31 - 2^24): the
// load returns zero without a memory access.  Used for the prefetch after the last block and
// for the pieces of a row past the head dim.
constexpr uint32_t kOutOfRange = 0x7FFFFFF0u;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

struct Rows {  // element strides of a (B, H, N, D) operand (last dim dense)
  long long b, h, n;
};
struct Vecs {  // element strides of a (B, H, D) operand
  long long b, h;
};

// Element type: the pair dot product v_dot2_f32_{bf16,f16} (a.lo*b.lo + a.hi*b.hi + c, fp32
// accumulate; products of two bf16 or two fp16 values are exact in fp32), the halves of a
// 32-bit pair as fp32, and the quiet-NaN pattern.
template <class T>
struct DElem;
template <>
struct DElem<__bf16> {
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                           __builtin_bit_cast(bf16x2, b), c, false);
  }
  static __device__ __forceinline__ float lo(uint32_t x) { return __uint_as_float(x << 16); }
  static __device__ __forceinline__ float hi(uint32_t x) { return __uint_as_float(x & 0xffff0000u); }
  static constexpr unsigned short kNaN = 0x7FC0;
};
template <>
struct DElem<_Float16> {
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c,
                                  false);
  }
  static __device__ __forceinline__ float lo(uint32_t x) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(x & 0xffffu));
  }
  static __device__ __forceinline__ float hi(uint32_t x) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(x >> 16));
  }
  static constexpr unsigned short kNaN = 0x7E00;
};

// Compile-time shape: element type T; kDP pieces of 32 head dims per key row (a lane holds
// 8 dims of each piece); kMaskD: the head dim D may be below 32 * kDP (a multiple of 8), and
// the 16-byte pieces at dims >= D are neither read nor written.
template <class T_, int kDP_, bool kMaskD_>
struct DShape {
  typedef T_ T;
  static constexpr int kDP = kDP_;
  static constexpr int kDm = 32 * kDP_;
  static constexpr bool kMaskD = kMaskD_;
};

// NaN marks results of invalid cache lengths.  The device pass is compiled with
// -fno-honor-nans, under which a floating-point select may drop a NaN operand, so these
// stores choose between bit patterns and write them through integer pointers.
template <class T>
__device__ __forceinline__ void store_o(T* p, float v, bool valid) {
  const unsigned short bits = __builtin_bit_cast(unsigned short, (T)v);
  *reinterpret_cast<unsigned short*>(p) = valid ? bits : DElem<T>::kNaN;
}
__device__ __forceinline__ void store_lse(float* p, float v, bool valid) {
  *reinterpret_cast<uint32_t*>(p) = valid ? __float_as_uint(v) : 0x7FC00000u;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const void* base, int nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, nbytes, 0x00020000);
}

__device__ __forceinline__ u32x4 load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

// Sum over the 4 lanes of a key column (one quad): xor 1 and xor 2 by DPP quad permutations.
__device__ __forceinline__ float quad_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));
  return x;
}

// This lane's share of one block of a wave: keys key0 + 16r (r < kKeysPerLane), each as kDP
// 16-byte pieces: piece p = dims 32p + 8c .. 32p + 8c + 7 (bytes 64p + 16c).  A wave
// instruction reads 16 rows x 64 contiguous bytes.
template <int kDP>
struct KV {
  u32x4 k[kKeysPerLane][kDP], v[kKeysPerLane][kDP];
};

// kb: the block's first key (wave-uniform); k_lane/v_lane: this lane's byte offset within a
// block, (l/4) * row + 16c; key r of the lane is 16r rows further.  A block that is not live
// loads from kOutOfRange (+ the lane part, still past num_records as an unsigned 32-bit
// offset); so does a piece past the head dim (bit p of pmask clear).
template <class Sh>
__device__ __forceinline__ void load_block(KV<Sh::kDP>& x, __amdgpu_buffer_rsrc_t kd,
                                           __amdgpu_buffer_rsrc_t vd, int krow, int vrow, int kb,
                                           bool live, int k_lane, int v_lane, uint32_t pmask) {
  const uint32_t ks = (uint32_t)__builtin_amdgcn_readfirstlane(live ? kb * krow : (int)kOutOfRange);
  const uint32_t vs = (uint32_t)__builtin_amdgcn_readfirstlane(live ? kb * vrow : (int)kOutOfRange);
#pragma unroll
  for (int r = 0; r < kKeysPerLane; ++r)
#pragma unroll
    for (int p = 0; p < Sh::kDP; ++p) {
      uint32_t ko = ks + (uint32_t)(k_lane + 16 * r * krow + 64 * p);
      uint32_t vo = vs + (uint32_t)(v_lane + 16 * r * vrow + 64 * p);
      if (Sh::kMaskD && !((pmask >> p) & 1u)) {
        ko = kOutOfRange;
        vo = kOutOfRange;
      }
      x.k[r][p] = load16(kd, ko);
      x.v[r][p] = load16(vd, vo);
    }
}

// (x.lo16, y.lo16) and (x.hi16, y.hi16): one head dim of two keys side by side (v_perm_b32).
__device__ __forceinline__ uint32_t pair_lo(uint32_t x, uint32_t y) {
  return __builtin_amdgcn_perm(y, x, 0x05040100u);
}
__device__ __forceinline__ uint32_t pair_hi(uint32_t x, uint32_t y) {
  return __builtin_amdgcn_perm(y, x, 0x07060302u);
}

// Online-softmax update of this key column's stream (m, l, o[8 kDP]) with the lane's keys of
// the block.
//   scores: q . k as dot2 of element pairs (q kept in the element type, exact products),
//   times scale*log2(e); even pieces accumulate in one sum, odd pieces in another;
//   o += p_r v_r + p_r+1 v_r+1 as dot2 of (p_r, p_r+1) with (v_r[d], v_r+1[d]) built by
//   v_perm; p is rounded to the element type for that product (as the forward kernel's P
//   operand), l sums it in fp32.
//   The running max is exact, so the largest weight of the stream is exactly 1.
//   o and l are rescaled only when some lane's max moved (wave-uniform test).
template <class Sh>
__device__ __forceinline__ void block_update(const KV<Sh::kDP>& x, const uint32_t (&qp)[4 * Sh::kDP],
                                             float scale_log2, int key0, int key_end, float& m,
                                             float& l, float (&o)[8 * Sh::kDP]) {
  typedef typename Sh::T T;
  float s[kKeysPerLane];
#pragma unroll
  for (int r = 0; r < kKeysPerLane; ++r) {
    float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
    for (int p = 0; p < Sh::kDP; p += 2)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc0 = DElem<T>::dot2(qp[4 * p + i], x.k[r][p][i], acc0);
        acc1 = DElem<T>::dot2(qp[4 * p + 4 + i], x.k[r][p + 1][i], acc1);
      }
    const float acc = quad_sum(acc0 + acc1) * scale_log2;
    s[r] = (key0 + 16 * r < key_end) ? acc : -INFINITY;
  }
  float m_new = m;
#pragma unroll
  for (int r = 0; r < kKeysPerLane; ++r) m_new = fmaxf(m_new, s[r]);
  const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
  if (__builtin_amdgcn_ballot_w64(m_new != m)) {
    const float alpha = exp2f(m - m_use);
    l *= alpha;
#pragma unroll
    for (int i = 0; i < 8 * Sh::kDP; ++i) o[i] *= alpha;
  }
#pragma unroll
  for (int r = 0; r < kKeysPerLane; r += 2) {
    const float p0 = exp2f(s[r] - m_use), p1 = exp2f(s[r + 1] - m_use);
    l += p0 + p1;
    T pe[2] = {(T)p0, (T)p1};
    const uint32_t pp = (uint32_t)__builtin_bit_cast(unsigned short, pe[0]) |
                        ((uint32_t)__builtin_bit_cast(unsigned short, pe[1]) << 16);
#pragma unroll
    for (int p = 0; p < Sh::kDP; ++p)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[8 * p + 2 * i] =
            DElem<T>::dot2(pp, pair_lo(x.v[r][p][i], x.v[r + 1][p][i]), o[8 * p + 2 * i]);
        o[8 * p + 2 * i + 1] =
            DElem<T>::dot2(pp, pair_hi(x.v[r][p][i], x.v[r + 1][p][i]), o[8 * p + 2 * i + 1]);
      }
  }
  m = m_new;
}

// The new token as one more key of the stream of key column 0 (lanes 0..3) of the calling
// wave; every other column sees it masked.  kn/vn: this lane's pieces of k_new and v_new
// (zero past the head dim).
template <class Sh>
__device__ __forceinline__ void new_key_update(const u32x4 (&kn)[Sh::kDP], const u32x4 (&vn)[Sh::kDP],
                                               const uint32_t (&qp)[4 * Sh::kDP], float scale_log2,
                                               bool mine, float& m, float& l,
                                               float (&o)[8 * Sh::kDP]) {
  typedef typename Sh::T T;
  float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
  for (int p = 0; p < Sh::kDP; p += 2)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc0 = DElem<T>::dot2(qp[4 * p + i], kn[p][i], acc0);
      acc1 = DElem<T>::dot2(qp[4 * p + 4 + i], kn[p + 1][i], acc1);
    }
  const float sc = mine ? quad_sum(acc0 + acc1) * scale_log2 : -INFINITY;
  const float m_new = fmaxf(m, sc);
  const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
  const float alpha = exp2f(m - m_use);
  const float pn = exp2f(sc - m_use);
  l = fmaf(l, alpha, pn);
#pragma unroll
  for (int p = 0; p < Sh::kDP; ++p)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[8 * p + 2 * i] = fmaf(pn, DElem<T>::lo(vn[p][i]), o[8 * p + 2 * i] * alpha);
      o[8 * p + 2 * i + 1] = fmaf(pn, DElem<T>::hi(vn[p][i]), o[8 * p + 2 * i + 1] * alpha);
    }
  m = m_new;
}

// Largest value over the 64 lanes of x when x is the same in the 4 lanes of each quad: row
// rotations by 4 and 8 (DPP) give every lane its 16-lane row's maximum, then the 4 rows are
// read as scalars.
__device__ __forceinline__ float wave_max_quads(float x) {
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x124, 0xF, 0xF, false)));
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF, false)));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Wave-wide max / sum (butterfly over the 64 lanes).
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// Partials of a split head (S > 1) are exchanged between workgroups on different XCDs, whose
// L2 caches are not coherent with each other: the partial stores are agent-scope relaxed
// atomic stores (written through to the device coherence point) and the merging loads use
// the same device-scope cache policy (sc1), the forms the compiler emits for agent-scope
// relaxed atomics.
typedef unsigned long long u64;
constexpr int kPolicyCoherent = 16;  // buffer-load cache policy bit sc1
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(__amdgpu_buffer_rsrc_t r, int off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kPolicyCoherent));
}

// Merge of the S partials (o_s[D], log2-domain lse_s; D + 1 floats each) of head bh by the
// kW waves of the workgroup that arrived last: wave w folds splits w, w + kW, ... in batches
// of kMergeBatch, every load of a batch in one memory round trip (one batch while
// S <= kW * kMergeBatch); lane = head dim (and head dim + 64 when kTwo).  The split weights
// 2^(lse_s - M) are formed in lanes 0..kMergeBatch-1 and read back as scalars; wave 0 folds
// the kW wave sums from LDS and writes O and LSE.
constexpr int kMaxSplits = 1024;
constexpr int kMergeBatch = 16;
template <class T, bool kTwo, int kW>
__device__ __forceinline__ void merge_splits(const float* part, int bh, int S, int D, int wave,
                                             int lane, bool valid, T* orow, float* lse_out,
                                             float* sh_m, float* sh_w, float (*sh_acc)[128]) {
  const int pstride = D + 1;
  // The head's S partials as one buffer: offsets past it (splits >= S) read as zero.
  const __amdgpu_buffer_rsrc_t pr = rows_rsrc(part + (long long)bh * S * pstride, S * pstride * 4);
  float M = -INFINITY, wt = 0.f, o0 = 0.f, o1 = 0.f;
  for (int s0 = wave; s0 < S; s0 += kW * kMergeBatch) {
    float x0[kMergeBatch], x1[kMergeBatch];
#pragma unroll
    for (int j = 0; j < kMergeBatch; ++j) {
      const int sj = s0 + j * kW;
      x0[j] = load_coherent(pr, (sj * pstride + lane) * 4);
      x1[j] = kTwo ? load_coherent(pr, (sj * pstride + 64 + lane) * 4) : 0.f;
    }
    const int sl = s0 + (lane & (kMergeBatch - 1)) * kW;  // the split whose lse this lane reads
    const float v = load_coherent(pr, (sl * pstride + D) * 4);
    const float lse_j = (lane < kMergeBatch && sl < S) ? v : -INFINITY;
    const float Mn = fmaxf(M, wave_max(lse_j));
    const float Mn_use = (Mn == -INFINITY) ? 0.f : Mn;
    const float a = exp2f(M - Mn_use);  // 0 before the first batch with a key
    wt *= a;
    o0 *= a;
    o1 *= a;
    const float w = exp2f(lse_j - Mn_use);  // 0 for splits past S or without keys
#pragma unroll
    for (int j = 0; j < kMergeBatch; ++j) {
      const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), j));
      wt += wj;
      o0 = fmaf(wj, x0[j], o0);
      if (kTwo) o1 = fmaf(wj, x1[j], o1);
    }
    M = Mn;
  }
  if (lane == 0) {
    sh_m[wave] = M;
    sh_w[wave] = wt;
  }
  sh_acc[wave][lane] = o0;
  if (kTwo) sh_acc[wave][64 + lane] = o1;
  __syncthreads();
  if (wave != 0) return;
  float Mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < kW; ++i) Mx = fmaxf(Mx, sh_m[i]);
  const float Mx_use = (Mx == -INFINITY) ? 0.f : Mx;
  float W = 0.f, a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int i = 0; i < kW; ++i) {
    const float f = exp2f(sh_m[i] - Mx_use);
    W = fmaf(f, sh_w[i], W);
    a0 = fmaf(f, sh_acc[i][lane], a0);
    if (kTwo) a1 = fmaf(f, sh_acc[i][64 + lane], a1);
  }
  if (lane < D) store_o<T>(orow + lane, W > 0.f ? a0 / W : 0.f, valid);
  if (kTwo && lane + 64 < D) store_o<T>(orow + 64 + lane, W > 0.f ? a1 / W : 0.f, valid);
  if (lse_out != nullptr && lane == 0)
    store_lse(lse_out, W > 0.f ? (Mx + log2f(W)) * kLn2 : -INFINITY, valid);
}

// kW waves per workgroup: kWavesWhole for one workgroup per head (S = 1: O and LSE written
// directly), kWavesSplit for S > 1 splits per head (part holds the partials, D + 1 floats each;
// arrive the heads' arrival words; tag this call's 48-bit tag).  kDense: every operand in the
// contiguous layout at D = kDm (caches (B, H, N_max, D), q, k_new, v_new, o (B, H, D)), whose
// offsets follow from bh; the stride arguments are not read.
//
// Argument order: the first 14 dwords are preloaded into SGPRs at wave launch
// (-amdgpu-kernarg-preload-count).  They hold what a workgroup needs for its first cache, q and
// length loads (the caches, cache_seqlens, q, the sizes) and the scale, so a dense workgroup
// issues them with no scalar load from the argument segment first; the other pointers are
// loaded while those are in flight.  Measured per graph-replayed step against the earlier order
// (q and the strides first, q loaded after the length): B1 H25 L1024 6.72 -> 5.90 us,
// B1 H16 L8192 10.66 -> 9.66 us, B8 H25 L1024 12.06 -> 11.12 us.
template <class Sh, int kW, bool kDense>
__global__ __launch_bounds__(64 * kW) void decode_kernel(
    typename Sh::T* Kc, typename Sh::T* Vc, const int* __restrict__ seqlens,
    const typename Sh::T* __restrict__ Q, int N_max, int S, int C, int H, float scale_log2,
    int D, u64* __restrict__ arrive, u64 tag, typename Sh::T* __restrict__ O,
    float* __restrict__ LSE, float* __restrict__ part, Vecs qs, Rows ks, Rows vs,
    const typename Sh::T* __restrict__ Kn, Vecs kns, const typename Sh::T* __restrict__ Vn,
    Vecs vns, Vecs os) {
  typedef typename Sh::T T;
  constexpr int kDP = Sh::kDP;
  constexpr int kDm = Sh::kDm;
  constexpr bool kSplit = kW == kWavesSplit;  // then S > 1
  static_assert(kW == kWavesSplit || kW == kWavesWhole, "two workgroup shapes");
  constexpr int kThreads = 64 * kW;
  constexpr int kBlockKeysW = kW * kWaveKeys;      // keys per workgroup per block
  constexpr int kStreams = kW * kGroups;           // softmax streams of the workgroup
  constexpr int kParts = kThreads / kDm;           // first-level merge: streams in kParts parts
  constexpr int kPerPart = kStreams / kParts;
  __shared__ float sh_o[kStreams][kDm + 1];        // +1: stream-major writes, dim-major reads
  __shared__ float sh_l[kStreams], sh_wm[kW];
  __shared__ float sh_po[kParts][kDm], sh_pm[kParts], sh_pl[kParts];
  __shared__ float sh_mm[kSplit ? kW : 1], sh_mw[kSplit ? kW : 1];  // merge_splits
  __shared__ float sh_macc[kSplit ? kW : 1][128];
  __shared__ int sh_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 2;  // key column within the wave
  const int c = lane & 3;   // dims 32p + 8c .. 32p + 8c + 7 of each piece p

  const int bh = blockIdx.x / S;
  const int s = blockIdx.x - bh * S;
  const int b = bh / H, h = bh - b * H;
  const bool append = Kn != nullptr;
  // Pieces of this lane inside the head dim: bit p set when dims 32p + 8c.. are below D.
  uint32_t pmask = 0;
#pragma unroll
  for (int p = 0; p < kDP; ++p) pmask |= (uint32_t)(!Sh::kMaskD || 32 * p + 8 * c < D) << p;

  const long long hrows = (long long)bh * N_max * kDm;  // dense: the head's first cache element
  T* Kh = Kc + (kDense ? hrows : b * ks.b + h * ks.h);
  T* Vh = Vc + (kDense ? hrows : b * vs.b + h * vs.h);
  const long long ksn = kDense ? kDm : ks.n, vsn = kDense ? kDm : vs.n;
  const int krow = (int)ksn * 2, vrow = (int)vsn * 2;
  const long long hvec = (long long)bh * kDm;  // dense: the head's q, k_new, v_new and o
  const int k_lane = g * krow + 16 * c;
  const int v_lane = g * vrow + 16 * c;
  const int c0 = s * C;
  int kb = c0 + wave * kWaveKeys;  // this wave's first block
  // The first block's loads go out before the cache length arrives from memory: over the whole
  // allocation (N_max rows, all addressable), with the rows at or past the length zeroed once
  // it is known (below), so no stale or appended-row value reaches the sums.
  KV<kDP> A;
  if (kb < min(c0 + C, N_max))
    load_block<Sh>(A, rows_rsrc(Kh, N_max * krow), rows_rsrc(Vh, N_max * vrow), krow, vrow, kb,
                   true, k_lane, v_lane, pmask);

  // q does not depend on the cache length: its loads go out before the length is read.
  uint32_t qp[4 * kDP];  // this lane's q pieces as element pairs (zero past the head dim)
  {
    const T* qh = Q + (kDense ? hvec : b * qs.b + h * qs.h);
#pragma unroll
    for (int p = 0; p < kDP; ++p) {
      u32x4 qv = {0, 0, 0, 0};
      if ((pmask >> p) & 1u) qv = *reinterpret_cast<const u32x4*>(qh + 32 * p + 8 * c);
#pragma unroll
      for (int i = 0; i < 4; ++i) qp[4 * p + i] = qv[i];
    }
  }

  const int Lc = seqlens ? seqlens[b] : N_max;  // valid cached rows
  // S > 1: this head's arrival word, read by wave 0 after its first cache, q and length loads
  // are issued (it is needed after the cache loop).
  u64* const aw = kSplit ? reinterpret_cast<u64*>(reinterpret_cast<char*>(arrive) +
                                                  (long long)bh * kArriveStride)
                         : nullptr;
  u64 aw_start = 0;
  if (kSplit) {
    if (wave == 0) aw_start = __hip_atomic_load(aw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_sched_barrier(0);
  }
  const bool valid = Lc >= 0 && Lc + (append ? 1 : 0) <= N_max;
  const int L = valid ? Lc + (append ? 1 : 0) : 0;  // keys attended
  const int c1 = min(c0 + C, L);
  const int Lr = valid ? Lc : 0;
  const __amdgpu_buffer_rsrc_t kd = rows_rsrc(Kh, Lr * krow);
  const __amdgpu_buffer_rsrc_t vd = rows_rsrc(Vh, Lr * vrow);
  // Arguments past the preloaded ones, needed once the first block is in: their loads go out
  // with the first block and the length rather than where they are used.
  asm volatile("" ::"s"(O), "s"(LSE), "s"(part), "s"(tag));

  // The new token: stored into the cache by the workgroup whose chunk holds row Lc.
  u32x4 k_app[kDP], v_app[kDP];
#pragma unroll
  for (int p = 0; p < kDP; ++p) {
    k_app[p] = u32x4{0, 0, 0, 0};
    v_app[p] = u32x4{0, 0, 0, 0};
  }
  const bool has_new = append && valid && Lc >= c0 && Lc < c0 + C;
  if (has_new) {
    const T* kn = Kn + (kDense ? hvec : b * kns.b + h * kns.h);
    const T* vn = Vn + (kDense ? hvec : b * vns.b + h * vns.h);
#pragma unroll
    for (int p = 0; p < kDP; ++p)
      if ((pmask >> p) & 1u) {
        k_app[p] = *reinterpret_cast<const u32x4*>(kn + 32 * p + 8 * c);
        v_app[p] = *reinterpret_cast<const u32x4*>(vn + 32 * p + 8 * c);
      }
    if (wave == 0 && g == 0) {
#pragma unroll
      for (int p = 0; p < kDP; ++p)
        if ((pmask >> p) & 1u) {
          *reinterpret_cast<u32x4*>(Kh + (long long)Lc * ksn + 32 * p + 8 * c) = k_app[p];
          *reinterpret_cast<u32x4*>(Vh + (long long)Lc * vsn + 32 * p + 8 * c) = v_app[p];
        }
    }
  }

  float m = -INFINITY, l = 0.f, o[8 * kDP];
#pragma unroll
  for (int i = 0; i < 8 * kDP; ++i) o[i] = 0.f;

  // Blocks of this wave: kb = c0 + 32*wave + 128*t.
  // Cached rows of this chunk: [c0, ce).  The appended row (Lc, if it falls in this chunk) is
  // not read from the cache; wave 0 folds it in after the loop.
  const int ce = min(c1, Lc);
  if (kb < ce) {  // then kb < min(c0 + C, N_max): A was loaded
    const int nblk = (ce - kb + kBlockKeysW - 1) / kBlockKeysW;  // this wave's blocks
#pragma unroll
    for (int r = 0; r < kKeysPerLane; ++r)
      if (kb + g + 16 * r >= Lr)
#pragma unroll
        for (int p = 0; p < kDP; ++p) {
          A.k[r][p] = u32x4{0, 0, 0, 0};
          A.v[r][p] = u32x4{0, 0, 0, 0};
        }
    // Two register sets used in turn: the next block's loads are in flight while one block
    // is computed, with no copies between the sets (a copy would wait for the loads).  Pairs
    // of blocks per iteration, one back edge and no exit inside the body, so at the top of an
    // iteration only A's loads are outstanding.  (A third set was measured slower: the
    // compiler then waits for two sets before the first block of an iteration.)
    KV<kDP> B;
    // The scheduling barriers keep each block's arithmetic after the loads issued before it:
    // left alone, the scheduler hoists the (independent) dot products of the next block, which
    // then wait for the loads just issued.
    for (int t = 0; t + 2 <= nblk; t += 2) {
      load_block<Sh>(B, kd, vd, krow, vrow, kb + kBlockKeysW, true, k_lane, v_lane, pmask);
      __builtin_amdgcn_sched_barrier(0);
      block_update<Sh>(A, qp, scale_log2, kb + g, ce, m, l, o);
      __builtin_amdgcn_sched_barrier(0);
      kb += kBlockKeysW;
      load_block<Sh>(A, kd, vd, krow, vrow, kb + kBlockKeysW, t + 2 < nblk, k_lane, v_lane, pmask);
      __builtin_amdgcn_sched_barrier(0);
      block_update<Sh>(B, qp, scale_log2, kb + g, ce, m, l, o);
      __builtin_amdgcn_sched_barrier(0);
      kb += kBlockKeysW;
    }
    if (nblk & 1) block_update<Sh>(A, qp, scale_log2, kb + g, ce, m, l, o);
  }
  if (has_new && wave == 0) new_key_update<Sh>(k_app, v_app, qp, scale_log2, g == 0, m, l, o);
  // Install this call's tag (count 0) unless a workgroup of the call already has; a failed
  // swap means exactly that, so its result is not needed.  Placed after the cache loop, where
  // every load (the word's first) has arrived: waiting for the word earlier would hold back
  // the loads issued after it.  It precedes this workgroup's count increment (same address,
  // program order).
  if (kSplit && wave == 0 && lane == 0 && (aw_start >> kTagShift) != tag) {
    u64 expected = aw_start;
    __hip_atomic_compare_exchange_strong(aw, &expected, tag << kTagShift, __ATOMIC_RELAXED,
                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // Merge the workgroup's 16 kW streams (16 key columns x kW waves) in two LDS rounds:
  //  1. each wave scales its streams once by 2^(m - M_w), M_w its largest stream maximum (row
  //     rotations and lane reads, no LDS), and writes them to LDS; thread t sums the streams
  //     of part t/kDm (kWavesPerPart whole waves) for head dim t%kDm, rescaling the waves'
  //     sums to the part's maximum;
  //  2. kDm threads fold the kParts partial sums with the log-sum-exp rule.
  // (Folding the 128 streams pairwise with their own maxima cost 16 exponentials and 32 more
  // LDS reads per thread, ~1 us per step at the bench shape.)
  constexpr int kWavesPerPart = kPerPart / kGroups;
  static_assert(kPerPart % kGroups == 0, "a part is whole waves");
  const int stream = wave * kGroups + g;
  const float Mw = wave_max_quads(m);
  const float sc = exp2f(m - ((Mw == -INFINITY) ? 0.f : Mw));  // 0 for a stream that saw no key
#pragma unroll
  for (int p = 0; p < kDP; ++p)
#pragma unroll
    for (int i = 0; i < 8; ++i) sh_o[stream][32 * p + 8 * c + i] = o[8 * p + i] * sc;
  if (c == 0) sh_l[stream] = l * sc;
  if (lane == 0) sh_wm[wave] = Mw;
  __syncthreads();
  {
    const int d = tid & (kDm - 1), pt = tid / kDm;
    float Mp = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < kWavesPerPart; ++ww) Mp = fmaxf(Mp, sh_wm[pt * kWavesPerPart + ww]);
    const float Mp_use = (Mp == -INFINITY) ? 0.f : Mp;
    float ot = 0.f, lt = 0.f;
#pragma unroll
    for (int ww = 0; ww < kWavesPerPart; ++ww) {
      const int w0 = (pt * kWavesPerPart + ww) * kGroups;
      float os_ = 0.f, ls = 0.f;
#pragma unroll
      for (int i = 0; i < kGroups; ++i) os_ += sh_o[w0 + i][d];
      if (d == 0)
#pragma unroll
        for (int i = 0; i < kGroups; ++i) ls += sh_l[w0 + i];
      const float f = kWavesPerPart == 1 ? 1.f : exp2f(sh_wm[pt * kWavesPerPart + ww] - Mp_use);
      ot = fmaf(f, os_, ot);
      lt = fmaf(f, ls, lt);
    }
    sh_po[pt][d] = ot;
    if (d == 0) {
      sh_pm[pt] = Mp;
      sh_pl[pt] = lt;
    }
  }
  __syncthreads();
  const bool writer = tid < kDm && !(Sh::kMaskD && tid >= D);  // thread d: head dim d
  if (!kSplit && !writer) return;
  if (writer) {
    const int d = tid;
    float M = -INFINITY;
#pragma unroll
    for (int i = 0; i < kParts; ++i) M = fmaxf(M, sh_pm[i]);
    const float M_use = (M == -INFINITY) ? 0.f : M;
    float lt = 0.f, ot = 0.f;
#pragma unroll
    for (int i = 0; i < kParts; ++i) {
      const float w = exp2f(sh_pm[i] - M_use);
      lt = fmaf(w, sh_pl[i], lt);
      ot = fmaf(w, sh_po[i][d], ot);
    }
    const float on = lt > 0.f ? ot / lt : 0.f;
    const float lse2 = lt > 0.f ? M + log2f(lt) : -INFINITY;
    if (!kSplit) {
      store_o<T>(O + (kDense ? hvec : b * os.b + h * os.h) + d, on, valid);
      if (LSE != nullptr && d == 0) store_lse(LSE + bh, lse2 * kLn2, valid);
      return;
    }
    float* pp = part + ((long long)bh * S + s) * (D + 1);
    store_coherent(pp + d, on);
    if (d == 0) store_coherent(pp + D, lse2);
  }
  if (!kSplit) return;
  // S > 1 (every thread of the workgroup is here): the partial is at the coherence point once
  // the writing waves' stores are acknowledged; then count the arrival.  The workgroup that
  // arrives last resets the word and merges the head.
  if (tid < kDm) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const u64 old = __hip_atomic_fetch_add(aw, (u64)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = (old & ((1ull << kTagShift) - 1)) == (u64)(S - 1);
    if (last) __hip_atomic_store(aw, (u64)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sh_last = last;
  }
  __syncthreads();
  if (!sh_last) return;
  asm volatile("" ::: "memory");  // the partial loads stay after the arrival count
  merge_splits<T, (kDm > 64), kW>(part, bh, S, D, wave, lane, valid,
                                  O + (kDense ? hvec : b * os.b + h * os.h),
                                  LSE != nullptr ? LSE + bh : nullptr, sh_mm, sh_mw, sh_macc);
}

// ---------------------------------------------------------------------------------------
// Host side.

// Splits for a cache of N_max rows of head dim D.  One 8-wave workgroup per head keeps 128 KiB
// of K/V loads in flight, enough to stream at HBM rate from one CU, so heads are not split
// while B*H exceeds half the CUs (no partials, no arrival count).  Measured (graph-replayed
// steps, us, unsplit -> split): 8 x 25 x 1024, D = 64: 11.97 -> 14.47; 16 x 12 x 1024, D = 128:
// 22.03 -> 25.47; at exactly half the CUs (B*H = 128) 4 x 32 x 2048, D = 64: 15.93 -> 15.83,
// 8 x 16 x 1024, D = 128: 17.13 -> 16.64 and 2 x 64 x 2048, D = 96: 27.48 -> 22.65 (one
// 222-VGPR workgroup per CU above D = 64, so half the CUs idle unsplit).  At or below half the
// CUs a head is split over 4-wave workgroups,
// two per CU, rounding down so that no slot runs two, and no split holds less than
// kSplitBytes of K and V (one key block at least).  Measured (graph-replayed steps, caches
// rotating through HBM; two-kernel split with 8-wave workgroups -> this one-kernel split):
// 1 x 16 heads x 8192 rows 12.3 -> 10.3 us, 1 x 25 x 1024 7.9 -> 6.5 us.  Chunks are a
// multiple of kSplitBlockKeys, no split is empty.
constexpr int kSplitBytes = 32 * 1024;
// Caches of fewer split blocks (1024 rows) are not split: at 1 x 25 heads x 512 rows one
// workgroup per head takes 6.1 us, the split 6.5 us; at 1024 rows the split wins.
constexpr int kMinSplitBlocks = 8;
constexpr int kSplitSlotsPerCu = 2;
static void choose_split(int BH, int N_max, int D, int cu_count, int max_splits, int* S_out,
                         int* C_out) {
  const int sblocks = std::max(1, (N_max + kSplitBlockKeys - 1) / kSplitBlockKeys);
  if (2 * BH <= cu_count && sblocks >= kMinSplitBlocks) {
    int S = std::max(1, kSplitSlotsPerCu * cu_count / BH);
    const int split_keys = std::max(kSplitBlockKeys, kSplitBytes / (4 * D));
    S = std::min(S, (N_max + split_keys - 1) / split_keys);
    S = std::max(1, std::min(std::min(S, max_splits), kMaxSplits));
    const int C = (sblocks + S - 1) / S * kSplitBlockKeys;
    S = (N_max + C - 1) / C;
    if (S > 1) {
      *S_out = S;
      *C_out = C;
      return;
    }
  }
  *S_out = 1;  // one chunk of the whole cache
  *C_out = std::max(1, (N_max + kBlockKeys - 1) / kBlockKeys) * kBlockKeys;
}

static bool rows_ok(const int64_t* st, int B, int H, int N_max, int D, Rows* out) {
  Rows r;
  r.b = B == 1 ? 0 : st[0];
  r.h = H == 1 ? 0 : st[1];
  r.n = N_max <= 1 ? D : st[2];
  if (st[3] != 1) return false;
  if (r.b < 0 || r.h < 0 || r.n < D || ((r.b | r.h | r.n) & 7)) return false;
  *out = r;
  return true;
}

// The contiguous layouts, as rows_ok and vecs_ok normalise them (strides of size-1 dimensions
// are 0).
static bool rows_dense(const Rows& r, int B, int H, int N_max, int D) {
  return r.b == (B == 1 ? 0 : (long long)H * N_max * D) &&
         r.h == (H == 1 ? 0 : (long long)N_max * D) && r.n == D;
}
static bool vecs_dense(const Vecs& v, int B, int H, int D) {
  return v.b == (B == 1 ? 0 : (long long)H * D) && v.h == (H == 1 ? 0 : (long long)D);
}

static bool vecs_ok(const int64_t* st, int B, int H, Vecs* out) {
  Vecs v;
  v.b = B == 1 ? 0 : st[0];
  v.h = H == 1 ? 0 : st[1];
  if (st[2] != 1) return false;
  if (v.b < 0 || v.h < 0 || ((v.b | v.h) & 7)) return false;
  *out = v;
  return true;
}

// O rows (D elements each) must not share elements: sorted by stride, each stride of a
// dimension of size > 1 is at least the span reached through the smaller one.
static bool vecs_overlap(const Vecs& v, int B, int H, int D) {
  long long st[2] = {v.b, v.h}, sz[2] = {B, H};
  if (st[1] < st[0]) {
    const long long t = st[0], z = sz[0];
    st[0] = st[1];
    sz[0] = sz[1];
    st[1] = t;
    sz[1] = z;
  }
  long long reach = D - 1;
  for (int i = 0; i < 2; ++i) {
    if (sz[i] == 1) continue;
    if (st[i] <= reach) return true;
    reach += (sz[i] - 1) * st[i];
  }
  return false;
}

// Scratch of tfgfa_decode_noalloc: the arrival words and split partials of one call, in a
// file-scope device array (one copy per GPU, held until the process ends) instead of a
// caller's workspace.  320 KiB holds every split the library chooses on a 256-CU device:
// B*H < 128 split heads (16 KiB of arrival words) and at most 2 workgroups per CU,
// B*H*S <= 512, times (D + 1) floats (133 KiB at D = 64, 264 KiB at D = 128).  The kernels get
// the array's device address, looked up once per device with hipGetSymbolAddress; the array's
// name itself is only a host-side stand-in.  Zero at load; every call leaves its arrival
// words at zero.
constexpr size_t kScratchBytes = 320 * 1024;
static __device__ __attribute__((aligned(256))) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
static std::once_flag g_scratch_once[kMaxDevices];
static void* g_scratch_ptr[kMaxDevices];
static int g_scratch_status[kMaxDevices];

// This device's scratch address (first call on a device: the symbol lookup, with that device
// current).  0, or the negated hipError_t of the failed lookup.
static int device_scratch(void** out) {
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return -(int)e;
  if (dev < 0 || dev >= kMaxDevices) return TFGFA_ERR_TOO_LARGE;
  std::call_once(g_scratch_once[dev], [dev]() {
    void* p = nullptr;
    const hipError_t se = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_status[dev] = se == hipSuccess ? 0 : -(int)se;
    g_scratch_ptr[dev] = se == hipSuccess ? p : nullptr;
  });
  if (g_scratch_status[dev] != 0) return g_scratch_status[dev];
  *out = g_scratch_ptr[dev];
  return TFGFA_OK;
}

// Bytes of one partial set (every head, one split) for head dim D: o_s[D] and lse_s.
static size_t split_bytes(long long bh, int D) { return (size_t)bh * (size_t)(D + 1) * sizeof(float); }

// Splits a workspace of `bytes` (arrival words `ab` bytes, then partial sets of `per_split`)
// holds; at least 1 (one split needs no workspace).
static int workspace_splits(size_t bytes, size_t ab, size_t per_split) {
  if (bytes <= ab) return 1;
  return (int)std::max((size_t)1, std::min((size_t)INT32_MAX, (bytes - ab) / per_split));
}
// Bytes of the arrival words at the start of a workspace: one per head, kArriveStride apart.
static size_t arrive_bytes(long long bh) { return ((size_t)bh * kArriveStride + 255) / 256 * 256; }

// A random nonzero 48-bit tag per call (splitmix64 over a process-wide counter and a seed from
// the clock and an address), so that no word left in memory by anything else is likely to
// carry it.
static u64 splitmix64(u64 x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}
static u64 next_tag() {
  static std::atomic<u64> counter{0};
  static const u64 seed =
      splitmix64((u64)std::chrono::steady_clock::now().time_since_epoch().count() ^
                 (u64)(uintptr_t)&counter);
  const u64 t = splitmix64(seed + counter.fetch_add(1, std::memory_order_relaxed)) &
                ((1ull << (64 - kTagShift)) - 1);
  return t ? t : 1;
}

// The decode step for one element type: argument checks, split choice, launches.
template <class T>
static int decode_step(const void* q, const int64_t* q_strides, void* k_cache,
                       const int64_t* k_strides, void* v_cache, const int64_t* v_strides,
                       const void* k_new, const int64_t* k_new_strides, const void* v_new,
                       const int64_t* v_new_strides, const int* cache_seqlens, void* o,
                       const int64_t* o_strides, float* lse, int B, int H, int N_max, int D,
                       float softmax_scale, void* workspace, size_t workspace_bytes,
                       void* hip_stream, bool use_scratch = false) {
  if (B < 0 || H < 0 || N_max < 0) return TFGFA_ERR_BAD_SHAPE;
  if (D < 8 || D > kMaxD || (D & 7)) return TFGFA_ERR_HEAD_DIM;
  if (!(softmax_scale > 0.f) || !isfinite(softmax_scale)) return TFGFA_ERR_SCALE;
  if ((k_new == nullptr) != (v_new == nullptr)) return TFGFA_ERR_NULL_POINTER;
  const bool append = k_new != nullptr;
  if (append && cache_seqlens == nullptr) return TFGFA_ERR_CACHE;
  if (B == 0 || H == 0) return TFGFA_OK;
  const long long bh = (long long)B * H;
  if (bh > INT32_MAX / 64) return TFGFA_ERR_TOO_LARGE;

  Rows ks, vs;
  Vecs qs, os, kns = {0, 0}, vns = {0, 0};
  if (!q_strides || !k_strides || !v_strides || !o_strides) return TFGFA_ERR_NULL_POINTER;
  if (append && (!k_new_strides || !v_new_strides)) return TFGFA_ERR_NULL_POINTER;
  if (!vecs_ok(q_strides, B, H, &qs) || !vecs_ok(o_strides, B, H, &os)) return TFGFA_ERR_STRIDE;
  if (!rows_ok(k_strides, B, H, N_max, D, &ks) || !rows_ok(v_strides, B, H, N_max, D, &vs))
    return TFGFA_ERR_STRIDE;
  if (append && (!vecs_ok(k_new_strides, B, H, &kns) || !vecs_ok(v_new_strides, B, H, &vns)))
    return TFGFA_ERR_STRIDE;
  if (vecs_overlap(os, B, H, D)) return TFGFA_ERR_STRIDE;
  // Cache rows are addressed with 32-bit buffer offsets (row index * row stride, plus a block).
  if (((long long)N_max + kBlockKeys) * ks.n * 2 > INT32_MAX ||
      ((long long)N_max + kBlockKeys) * vs.n * 2 > INT32_MAX)
    return TFGFA_ERR_TOO_LARGE;

  if (!q || !k_cache || !v_cache || !o) return TFGFA_ERR_NULL_POINTER;
  if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)o |
       (uintptr_t)k_new | (uintptr_t)v_new | (uintptr_t)workspace) & 15u)
    return TFGFA_ERR_ALIGNMENT;
  if (((uintptr_t)lse | (uintptr_t)cache_seqlens) & 3u) return TFGFA_ERR_ALIGNMENT;

  int cu = 0;
  const int st = tfgfa_device_info(&cu, nullptr, nullptr, 0);
  if (st != TFGFA_OK) return st;
  const size_t per_split = split_bytes(bh, D);
  const size_t ab = arrive_bytes(bh);
  if (use_scratch) {
    // The scratch is the workspace: the split is limited to what it holds, exactly as for a
    // caller's workspace of that size.
    const int sst = device_scratch(&workspace);
    if (sst != TFGFA_OK) return sst;
    workspace_bytes = kScratchBytes;
  }
  int S, C;
  choose_split((int)bh, N_max, D, cu,
               workspace_splits(workspace ? workspace_bytes : 0, ab, per_split), &S, &C);
  if (bh * S > INT32_MAX) return TFGFA_ERR_TOO_LARGE;

  const hipStream_t stream = (hipStream_t)hip_stream;
  const float scale_log2 = softmax_scale * kLog2e;
  const T* qt = static_cast<const T*>(q);
  T* kc = static_cast<T*>(k_cache);
  T* vc = static_cast<T*>(v_cache);
  const T* knt = static_cast<const T*>(k_new);
  const T* vnt = static_cast<const T*>(v_new);
  T* ot = static_cast<T*>(o);
  // Workspace: arrival words, then the partials (S > 1 only).
  u64* arrive = static_cast<u64*>(workspace);
  float* ws = S > 1 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + ab) : nullptr;
  const u64 tag = S > 1 ? next_tag() : 0;
  const dim3 grid((unsigned)(bh * S));
  // Dense: every operand in the contiguous layout (caches (B, H, N_max, D), q, k_new, v_new and
  // o (B, H, D)) at D = 64 or 128, as KVCache allocates them; those instances read no strides.
  const bool dense = (D == 64 || D == 128) && rows_dense(ks, B, H, N_max, D) &&
                     rows_dense(vs, B, H, N_max, D) && vecs_dense(qs, B, H, D) &&
                     vecs_dense(os, B, H, D) &&
                     (!append || (vecs_dense(kns, B, H, D) && vecs_dense(vns, B, H, D)));
#define TFGFA_DECODE_LAUNCH_W(kDP, kMask, kW, kDn)                                            \
  hipLaunchKernelGGL((decode_kernel<DShape<T, kDP, kMask>, kW, kDn>), grid, dim3(64 * kW), 0, \
                     stream, kc, vc, cache_seqlens, qt, N_max, S, C, H, scale_log2, D, arrive, \
                     tag, ot, lse, ws, qs, ks, vs, knt, kns, vnt, vns, os)
#define TFGFA_DECODE_LAUNCH(kDP, kMask, kDn)                 \
  do {                                                       \
    if (S > 1)                                               \
      TFGFA_DECODE_LAUNCH_W(kDP, kMask, kWavesSplit, kDn);   \
    else                                                     \
      TFGFA_DECODE_LAUNCH_W(kDP, kMask, kWavesWhole, kDn);   \
  } while (0)
  if (D == 64 && dense)
    TFGFA_DECODE_LAUNCH(2, false, true);
  else if (D == 64)
    TFGFA_DECODE_LAUNCH(2, false, false);
  else if (D < 64)
    TFGFA_DECODE_LAUNCH(2, true, false);
  else if (D == 128 && dense)
    TFGFA_DECODE_LAUNCH(4, false, true);
  else if (D == 128)
    TFGFA_DECODE_LAUNCH(4, false, false);
  else
    TFGFA_DECODE_LAUNCH(4, true, false);
#undef TFGFA_DECODE_LAUNCH
#undef TFGFA_DECODE_LAUNCH_W
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return -(int)e;
  return TFGFA_OK;
}

// A plain streaming read: the floor a decode step's cache reads are measured against.  Workgroup
// w reads 16-B words [w * per_wg, (w + 1) * per_wg) of the buffer (kReadUnroll loads in flight
// per thread), folds them with xor and writes one word to sink[w % kSinkWords], so that no load
// can be dropped; the sink's contents mean nothing.
constexpr int kReadUnroll = 8;
constexpr int kSinkWords = 4096;
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ p, long long n16,
                                                          int per_wg, uint32_t* __restrict__ sink) {
  const long long base = (long long)blockIdx.x * per_wg;
  uint32_t acc = 0;
  for (int i0 = 0; i0 < per_wg; i0 += 256 * kReadUnroll) {
    u32x4 v[kReadUnroll];
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) {
      const int i = i0 + u * 256 + (int)threadIdx.x;
      const long long j = base + i;
      v[u] = (i < per_wg && j < n16) ? p[j] : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o);
  __shared__ uint32_t wave_acc[4];
  if ((threadIdx.x & 63) == 0) wave_acc[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0)
    sink[blockIdx.x % kSinkWords] = wave_acc[0] ^ wave_acc[1] ^ wave_acc[2] ^ wave_acc[3];
}

}  // namespace tfgfa_dec

extern "C" int tfgfa_stream_read(const void* p, size_t bytes, void* sink, void* hip_stream) {
  using namespace tfgfa_dec;
  if (bytes == 0) return TFGFA_OK;
  if (p == nullptr || sink == nullptr) return TFGFA_ERR_NULL_POINTER;
  if ((((uintptr_t)p) & 15u) || (bytes & 15u) || (((uintptr_t)sink) & 3u)) return TFGFA_ERR_ALIGNMENT;
  const long long n16 = (long long)(bytes / 16);
  // At least 256 workgroups (every CU streams), each reading at least 32 KiB, at most 4096.
  const long long wg = std::max(256LL, std::min(4096LL, n16 / 2048));
  const long long per_wg = (n16 + wg - 1) / wg;
  if (per_wg > INT32_MAX) return TFGFA_ERR_TOO_LARGE;
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)wg), dim3(256), 0, (hipStream_t)hip_stream,
                     static_cast<const u32x4*>(p), n16, (int)per_wg, static_cast<uint32_t*>(sink));
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? TFGFA_OK : -(int)e;
}

extern "C" size_t tfgfa_decode_workspace_size(int B, int H, int N_max, int D) {
  using namespace tfgfa_dec;
  if (B <= 0 || H <= 0 || N_max <= 0 || D < 8 || D > kMaxD || (D & 7)) return 0;
  // One partial per 128 cache rows: an upper bound on the splits of any block size >= 128,
  // so the size does not change with the kernel's tiling.
  const size_t blocks = ((size_t)N_max + kWorkspaceRows - 1) / kWorkspaceRows;
  return arrive_bytes((long long)B * H) + split_bytes((long long)B * H, D) * blocks;
}

extern "C" int tfgfa_decode_splits(int B, int H, int N_max, int D, int cu_count,
                                   size_t workspace_bytes) {
  using namespace tfgfa_dec;
  if (B <= 0 || H <= 0 || N_max <= 0 || D < 8 || D > kMaxD || (D & 7) || cu_count <= 0) return 0;
  const long long bh = (long long)B * H;
  if (bh > INT32_MAX) return 0;
  int S, C;
  choose_split((int)bh, N_max, D, cu_count,
               workspace_splits(workspace_bytes, arrive_bytes(bh), split_bytes(bh, D)), &S, &C);
  return S;
}

extern "C" size_t tfgfa_decode_scratch_bytes(void) { return tfgfa_dec::kScratchBytes; }

extern "C" size_t tfgfa_decode_workspace_bytes(int B, int H, int N_max) {
  return tfgfa_decode_workspace_size(B, H, N_max, tfgfa_dec::kD);
}

extern "C" int tfgfa_decode_bf16(const void* q, const int64_t* q_strides, void* k_cache,
                                 const int64_t* k_strides, void* v_cache,
                                 const int64_t* v_strides, const void* k_new,
                                 const int64_t* k_new_strides, const void* v_new,
                                 const int64_t* v_new_strides, const int* cache_seqlens, void* o,
                                 const int64_t* o_strides, float* lse, int B, int H, int N_max,
                                 int D, float softmax_scale, void* workspace,
                                 size_t workspace_bytes, void* hip_stream) {
  if (B < 0 || H < 0 || N_max < 0) return TFGFA_ERR_BAD_SHAPE;
  if (D != tfgfa_dec::kD) return TFGFA_ERR_HEAD_DIM;
  return tfgfa_dec::decode_step<__bf16>(q, q_strides, k_cache, k_strides, v_cache, v_strides,
                                           k_new, k_new_strides, v_new, v_new_strides,
                                           cache_seqlens, o, o_strides, lse, B, H, N_max, D,
                                           softmax_scale, workspace, workspace_bytes, hip_stream);
}

extern "C" int tfgfa_decode(const void* q, const int64_t* q_strides, void* k_cache,
                            const int64_t* k_strides, void* v_cache, const int64_t* v_strides,
                            const void* k_new, const int64_t* k_new_strides, const void* v_new,
                            const int64_t* v_new_strides, const int* cache_seqlens, void* o,
                            const int64_t* o_strides, float* lse, int B, int H, int N_max, int D,
                            int dtype, float softmax_scale, void* workspace,
                            size_t workspace_bytes, void* hip_stream) {
  if (dtype == TFGFA_DTYPE_BF16)
    return tfgfa_dec::decode_step<__bf16>(q, q_strides, k_cache, k_strides, v_cache,
                                             v_strides, k_new, k_new_strides, v_new,
                                             v_new_strides, cache_seqlens, o, o_strides, lse, B, H,
                                             N_max, D, softmax_scale, workspace, workspace_bytes,
                                             hip_stream);
  if (dtype == TFGFA_DTYPE_F16)
    return tfgfa_dec::decode_step<_Float16>(q, q_strides, k_cache, k_strides, v_cache,
                                               v_strides, k_new, k_new_strides, v_new,
                                               v_new_strides, cache_seqlens, o, o_strides, lse, B,
                                               H, N_max, D, softmax_scale, workspace,
                                               workspace_bytes, hip_stream);
  return TFGFA_ERR_DTYPE;
}

extern "C" int tfgfa_decode_noalloc(const void* q, const int64_t* q_strides, void* k_cache,
                                    const int64_t* k_strides, void* v_cache,
                                    const int64_t* v_strides, const void* k_new,
                                    const int64_t* k_new_strides, const void* v_new,
                                    const int64_t* v_new_strides, const int* cache_seqlens,
                                    void* o, const int64_t* o_strides, float* lse, int B, int H,
                                    int N_max, int D, int dtype, float softmax_scale,
                                    void* hip_stream) {
  if (dtype == TFGFA_DTYPE_BF16)
    return tfgfa_dec::decode_step<__bf16>(q, q_strides, k_cache, k_strides, v_cache,
                                             v_strides, k_new, k_new_strides, v_new,
                                             v_new_strides, cache_seqlens, o, o_strides, lse, B, H,
                                             N_max, D, softmax_scale, nullptr, 0, hip_stream,
                                             true);
  if (dtype == TFGFA_DTYPE_F16)
    return tfgfa_dec::decode_step<_Float16>(q, q_strides, k_cache, k_strides, v_cache,
                                               v_strides, k_new, k_new_strides, v_new,
                                               v_new_strides, cache_seqlens, o, o_strides, lse, B,
                                               H, N_max, D, softmax_scale, nullptr, 0, hip_stream,
                                               true);
  return TFGFA_ERR_DTYPE;
}
