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
//   32 query rows and walks the key/value sequence in 64-key tiles staged in LDS, shared
//   by the 4 waves.  Tiles wholly above the causal diagonal are never loaded (per
//   workgroup) or computed (per wave); only tiles that cross the diagonal or the sequence
//   end apply an element mask.  Workgroups are issued heaviest query block first.
//
// MFMA chaining without an LDS round trip (v_mfma_f32_32x32x16_bf16, fp32 accumulate)
//   S^T = K . Q^T  : A = K tile rows (32 keys x 16 d), B = Q^T (16 d x 32 queries).
//                    Accumulator lane l holds query l%32 and 16 of the 32 keys, so a row's
//                    max/sum is an in-lane reduction plus one exchange with lane l^32.
//   O^T = V^T . P^T: B = P^T comes straight from the S^T accumulator registers (the
//                    contraction order over keys is relabelled to match), A = V^T is read
//                    from a transposed V tile in LDS.  O^T's lane l again holds query l%32.
//   Lane layouts assumed for 32x32x16 (K = 16 per instruction):
//     A[i][k]: lane = i + 32*(k/8), element k%8        B[k][j]: lane = j + 32*(k/8), element k%8
//     D[i][j]: lane = j + 32*((i/4)%2), register 4*(i/8) + i%4
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
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kD = 64;                      // head dimension (the only compiled one)
constexpr int kWaves = 4;                   // waves per workgroup
constexpr int kThreads = kWaves * 64;       // 256
constexpr int kWaveRows = 32;               // query rows per wave (one MFMA column block)
constexpr int kBlockRows = kWaves * kWaveRows;  // 128 query rows per workgroup
constexpr int kTileKeys = 64;               // keys per K/V tile
constexpr int kKRowBytes = kD * 2;          // 128 B per K row in LDS
constexpr int kKTileBytes = kTileKeys * kKRowBytes;  // 8 KiB
constexpr int kVtStride = kTileKeys + 4;    // bf16 per V^T row: 136 B, keeps b64 reads 8-B aligned
constexpr int kVtTileBytes = kD * kVtStride * 2;     // 8.5 KiB
constexpr int kSmemBytes = 2 * kKTileBytes + 2 * kVtTileBytes;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Buffer resource over one head's (N, 64) bf16 rows: loads at byte offsets >= N*128 return
// zero, which is how tiles and query blocks are zero-filled past the sequence end without a
// branch.  The whole offset is kept in the VGPR operand so the range check covers all of it.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t head_rsrc(const __bf16* base, int N) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<__bf16*>(base), (short)0, N * kKRowBytes,
                                           0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}

// Loads of one K tile (2 x 16 B per thread) and one V tile (2 rows x 16 B per thread) into
// registers.
struct TileRegs {
  uint4 k[2];
  uint4 v[2];
};

__device__ __forceinline__ void load_tile(TileRegs& r, __amdgpu_buffer_rsrc_t kr,
                                          __amdgpu_buffer_rsrc_t vr, int k0, int tid) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int ci = tid + kThreads * i;  // 16-B chunk index in the 64 x 64 tile
    const int key = ci >> 3;
    const int ch = ci & 7;
    r.k[i] = buf_load16(kr, (k0 + key) * kKRowBytes + ch * 16);
  }
  const int ch = tid & 7;   // d chunk: d = 8*ch .. 8*ch+7
  const int kp = tid >> 3;  // key pair: keys 2*kp, 2*kp+1
#pragma unroll
  for (int i = 0; i < 2; ++i) r.v[i] = buf_load16(vr, (k0 + 2 * kp + i) * kKRowBytes + ch * 16);
}

// K rows go to LDS with their 16-B chunks XOR-swizzled by (key & 7), so the 32 lanes of an
// A-operand read (32 rows, one logical chunk) spread over all banks.  V is written
// transposed (V^T[d][key]) so the P.V A-operand is two 8-B reads of 4 consecutive keys.
__device__ __forceinline__ void store_tile(const TileRegs& r, unsigned char* sK, unsigned char* sVt,
                                           int tid) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int ci = tid + kThreads * i;
    const int key = ci >> 3;
    const int ch = ci & 7;
    *reinterpret_cast<uint4*>(sK + key * kKRowBytes + ((ch ^ (key & 7)) << 4)) = r.k[i];
  }
  const int ch = tid & 7;
  const int kp = tid >> 3;
  const uint32_t a[4] = {r.v[0].x, r.v[0].y, r.v[0].z, r.v[0].w};  // key 2kp,   d = 8ch..
  const uint32_t b[4] = {r.v[1].x, r.v[1].y, r.v[1].z, r.v[1].w};  // key 2kp+1, d = 8ch..
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t even = (a[w] & 0xffffu) | (b[w] << 16);          // d = 8ch + 2w
    const uint32_t odd = (a[w] >> 16) | (b[w] & 0xffff0000u);       // d = 8ch + 2w + 1
    const int d = 8 * ch + 2 * w;
    *reinterpret_cast<uint32_t*>(sVt + (d * kVtStride) * 2 + kp * 4) = even;
    *reinterpret_cast<uint32_t*>(sVt + ((d + 1) * kVtStride) * 2 + kp * 4) = odd;
  }
}

__global__ __launch_bounds__(kThreads, 2) void fwd_kernel(
    const __bf16* __restrict__ Q, const __bf16* __restrict__ K, const __bf16* __restrict__ V,
    __bf16* __restrict__ O, float* __restrict__ LSE, int BH, int N, int nQB, float scale_log2,
    int causal) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[kSmemBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r32 = lane & 31;
  const int h = lane >> 5;

  // Heaviest (last) query blocks first: with causal masking block qb needs qb+1 key blocks.
  const int bid = blockIdx.x;
  const int qb = nQB - 1 - bid / BH;
  const int bh = bid % BH;

  const size_t head_off = (size_t)bh * N * kD;
  const __bf16* Qh = Q + head_off;
  const __bf16* Kh = K + head_off;
  const __bf16* Vh = V + head_off;

  const int q0 = qb * kBlockRows + wave * kWaveRows;  // first query row of this wave
  const int qrow = q0 + r32;                          // this lane's query row

  const __amdgpu_buffer_rsrc_t q_rsrc = head_rsrc(Qh, N);
  const __amdgpu_buffer_rsrc_t k_rsrc = head_rsrc(Kh, N);
  const __amdgpu_buffer_rsrc_t v_rsrc = head_rsrc(Vh, N);

  // Q^T operand for S^T = K Q^T: lane holds Q[qrow][16c + 8h .. 16c + 8h + 7], c = 0..3
  // (zero for rows past the end).
  bf16x8 qop[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    qop[c] = __builtin_bit_cast(bf16x8, buf_load16(q_rsrc, qrow * kKRowBytes + 32 * c + 16 * h));

  const int kv_end = causal ? min(N, (qb + 1) * kBlockRows) : N;
  const int nT = (kv_end + kTileKeys - 1) / kTileKeys;

  f32x16 o0, o1;  // O^T accumulators: d = 0..31 and d = 32..63
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    o0[t] = 0.f;
    o1[t] = 0.f;
  }
  float m_run = -INFINITY;  // running max of scale*log2e*s
  float l_run = 0.f;        // running sum of exp2(scale*log2e*s - m_run)

  TileRegs regs;
  load_tile(regs, k_rsrc, v_rsrc, 0, tid);
  store_tile(regs, smem, smem + 2 * kKTileBytes, tid);
  __syncthreads();

  for (int j = 0; j < nT; ++j) {
    const int buf = j & 1;
    const int k0 = j * kTileKeys;
    if (j + 1 < nT) load_tile(regs, k_rsrc, v_rsrc, k0 + kTileKeys, tid);

    const bool active = (q0 < N) && !(causal && k0 > q0 + kWaveRows - 1);
    if (active) {
      const unsigned char* sK = smem + buf * kKTileBytes;
      const unsigned char* sVt = smem + 2 * kKTileBytes + buf * kVtTileBytes;

      // S^T for keys k0 + [0,32) (s0) and k0 + [32,64) (s1).
      f32x16 s0, s1;
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        s0[t] = 0.f;
        s1[t] = 0.f;
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int sw = ((2 * c + h) ^ (r32 & 7)) << 4;
        const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(sK + r32 * kKRowBytes + sw);
        const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(sK + (32 + r32) * kKRowBytes + sw);
        s0 = mfma32(a0, qop[c], s0);
        s1 = mfma32(a1, qop[c], s1);
      }

      // Element mask only where the tile crosses the diagonal or the sequence end.
      const bool need_mask = (causal && k0 + kTileKeys - 1 > q0) || (k0 + kTileKeys > N);
      if (need_mask) {
#pragma unroll
        for (int t = 0; t < 16; ++t) {
          const int key = k0 + 8 * (t >> 2) + 4 * h + (t & 3);
          if ((causal && key > qrow) || key >= N) s0[t] = -INFINITY;
          if ((causal && key + 32 > qrow) || key + 32 >= N) s1[t] = -INFINITY;
        }
      }

      float mx = s0[0];
#pragma unroll
      for (int t = 1; t < 16; ++t) mx = fmaxf(mx, s0[t]);
#pragma unroll
      for (int t = 0; t < 16; ++t) mx = fmaxf(mx, s1[t]);
      mx = fmaxf(mx, __shfl_xor(mx, 32));

      const float m_new = fmaxf(m_run, mx * scale_log2);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      float sum = 0.f;
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        s0[t] = __builtin_amdgcn_exp2f(fmaf(s0[t], scale_log2, -m_new));
        sum += s0[t];
      }
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        s1[t] = __builtin_amdgcn_exp2f(fmaf(s1[t], scale_log2, -m_new));
        sum += s1[t];
      }
      sum += __shfl_xor(sum, 32);
      l_run = l_run * alpha + sum;
      m_run = m_new;
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        o0[t] *= alpha;
        o1[t] *= alpha;
      }

      // P^T operands: chunk c4 covers keys 16*c4 .. 16*c4+15 of the tile; this lane's 8
      // values are accumulator registers 8*(c4&1) .. +7 of s0 (c4 < 2) or s1.
      bf16x8 pb[4];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pb[0][e] = (__bf16)s0[e];
        pb[1][e] = (__bf16)s0[8 + e];
        pb[2][e] = (__bf16)s1[e];
        pb[3][e] = (__bf16)s1[8 + e];
      }

      // O^T += V^T P^T.  Element e of chunk c4 in lane half h is key
      //   16*c4 + 8*(e/4) + 4*h + e%4,
      // i.e. two runs of 4 consecutive keys read from V^T row d.
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) {
        const int koff = 16 * c4 + 4 * h;
        {
          const unsigned char* row = sVt + (r32 * kVtStride + koff) * 2;
          const uint2 lo = *reinterpret_cast<const uint2*>(row);
          const uint2 hi = *reinterpret_cast<const uint2*>(row + 16);
          const bf16x8 va = __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
          o0 = mfma32(va, pb[c4], o0);
        }
        {
          const unsigned char* row = sVt + ((32 + r32) * kVtStride + koff) * 2;
          const uint2 lo = *reinterpret_cast<const uint2*>(row);
          const uint2 hi = *reinterpret_cast<const uint2*>(row + 16);
          const bf16x8 va = __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
          o1 = mfma32(va, pb[c4], o1);
        }
      }
    }

    if (j + 1 < nT) {
      const int nb = (j + 1) & 1;
      store_tile(regs, smem + nb * kKTileBytes, smem + 2 * kKTileBytes + nb * kVtTileBytes, tid);
    }
    __syncthreads();
  }

  if (qrow < N) {
    const float inv_l = 1.0f / l_run;
    __bf16* orow = O + head_off + (size_t)qrow * kD;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      bf16x4 lo4, hi4;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        lo4[r] = (__bf16)(o0[4 * g + r] * inv_l);
        hi4[r] = (__bf16)(o1[4 * g + r] * inv_l);
      }
      *reinterpret_cast<bf16x4*>(orow + 8 * g + 4 * h) = lo4;
      *reinterpret_cast<bf16x4*>(orow + 32 + 8 * g + 4 * h) = hi4;
    }
    if (LSE != nullptr && h == 0) {
      LSE[(size_t)bh * N + qrow] = (m_run + __builtin_amdgcn_logf(l_run)) * kLn2;
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
