/*
 * tfgfa.h - C ABI of the MI355X (gfx950) causal FlashAttention forward.
 *
 * This is the drop-in boundary for the reference's single hot path:
 *
 *   custom_flash_attn.forward(Q, K_mat, V) -> O
 *     reference: src/cpp/torch_bind.cpp:21-49 (pybind11/libtorch binding)
 *             -> src/cpp/v1.cu:4-38 (host launcher flashattention_forward<T>)
 *             -> src/cpp/headers/v1_implementation.hpp:12-171 (device kernel)
 *
 * The reference binds the launcher through a C++ template declaration
 * (torch_bind.cpp:9-11); here the same step is a plain C function taking
 * device pointers, sizes and a HIP stream, with no torch types, so that any
 * FFI (pybind11, ctypes, cgo ...) can bind it.
 *
 * Conventions shared by every entry point:
 *  - Q, K, V, O are (B, H, N, D) bfloat16 tensors in device memory, 16-byte
 *    aligned.  tfgfa_fwd_bf16 takes them contiguous (strides H*N*D, N*D, D, 1),
 *    the layout torch_bind.cpp:27-31 assumes (size(0..2) read as B, H, N;
 *    O = empty_like(Q)); tfgfa_fwd_bf16_strided takes any strides that keep
 *    the last dimension dense.
 *  - LSE, when requested, is a contiguous (B, H, N) float32 tensor holding the
 *    natural-log log-sum-exp of each row's scaled, masked scores:
 *        LSE[b,h,i] = log( sum_{j <= i} exp(scale * q_i . k_j) )
 *    (the lse_i of src/py/triton_implementation.py:153-154, which the
 *    reference computes but never stores, :162-166).
 *  - The caller owns every buffer; the library allocates no device memory.
 *  - Return value: 0 on success, > 0 invalid argument (checked before any HIP
 *    call, so argument errors are reported identically with or without a GPU),
 *    < 0 the negated hipError_t of a failed HIP call.
 *  - Calls are reentrant; launches are asynchronous on the given stream.
 *
 * Numeric range of the forward (tfgfa_fwd, tfgfa_fwd_bf16, tfgfa_fwd_bf16_strided).
 * Scores and sums are fp32.  The softmax offset of a row moves lazily: only when the
 * probabilities taken against the current offset grow too large (bf16: a lane's running
 * sum of them would pass 2^64, or, in a wave's last 32-key half, a probability would pass
 * 2^60; fp16: a probability rounded to fp16 would be infinite, i.e. above 65504, or, in a
 * wave's last half, would pass 2^15) does it jump to the row's running maximum (the
 * reference moves it on every tile, src/cpp/headers/v1_implementation.hpp:121-128).  So the
 * fp32 accumulators of P.V and of the sums stay finite while
 *     max|V| < 2^62          (bf16, any N_k; the reference's exact offset allows
 *                             N_k * max|V| < 2^128),
 *     N_k * max|V| < 2^112   (fp16; always true, fp16 values are below 2^16).
 * Past that bound a bf16 row may come out inf or NaN where the exact-offset reference
 * stays finite.  LSE is not affected.
 */
#ifndef TFGFA_H
#define TFGFA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 8: tfgfa_decode_splits, tfgfa_decode_scratch_bytes and tfgfa_stream_read added;
 * tfgfa_decode_noalloc splits only as far as its scratch holds instead of returning
 * TFGFA_ERR_SCRATCH. */
#define TFGFA_ABI_VERSION 8

/* Status codes (> 0: invalid argument). */
#define TFGFA_OK                 0
#define TFGFA_ERR_NULL_POINTER   1  /* q, k, v or o is NULL                          */
#define TFGFA_ERR_BAD_SHAPE      2  /* B, H or N negative                            */
#define TFGFA_ERR_HEAD_DIM       3  /* D not a multiple of 8 in [8, 128] (not 64: tfgfa_decode_bf16) */
#define TFGFA_ERR_SCALE          4  /* softmax_scale not finite or not > 0           */
#define TFGFA_ERR_CAUSAL_FLAG    5  /* causal is neither 0 nor 1                     */
#define TFGFA_ERR_TOO_LARGE      6  /* grid or element count exceeds the limits      */
#define TFGFA_ERR_ALIGNMENT      7  /* q/k/v/o not 16-byte aligned or lse not 4-byte */
#define TFGFA_ERR_STRIDE         8  /* strides outside what the entry point takes         */
#define TFGFA_ERR_CACHE          9  /* k_new/v_new given without cache_seqlens            */
#define TFGFA_ERR_DTYPE         10  /* dtype is not a TFGFA_DTYPE_* value                 */
#define TFGFA_ERR_SCRATCH       11  /* reserved: tfgfa_decode_noalloc limits its split to
                                       its scratch and no longer returns it                */

/* Element types of q, k, v, o (fp32 accumulation and softmax either way). */
#define TFGFA_DTYPE_BF16 0
#define TFGFA_DTYPE_F16  1

/*
 * Attention forward, bf16 in / bf16 out, fp32 accumulation and softmax.
 *
 *   O[b,h,i,:] = sum_j softmax_j(scale * Q[b,h,i,:] . K[b,h,j,:]) * V[b,h,j,:]
 *   with j <= i when causal == 1 (top-left aligned, diagonal included), all j otherwise.
 *
 * Replaces flashattention_forward<__nv_bfloat16>(O, Q, K_mat, V, seq_len,
 * batch_size, num_heads) (src/cpp/v1.cu:4-38, instantiated :40-42), whose
 * scale is fixed to 1/sqrt(64) (v1.cu:16) and whose launch goes to the legacy
 * default stream (v1.cu:33-34).  D: a multiple of 8 up to 128 (the reference
 * compiles 64 only, common_types.hpp:33); tfgfa_fwd with dtype bf16,
 * N_q = N_k.  Here the scale is explicit (pass 0.125 for the reference's
 * behaviour), `lse` may be NULL (the reference's O-only call; a kernel built
 * without the LSE's running sum then runs, O bitwise the same), and
 * `hip_stream` (a hipStream_t, NULL = default stream) is the stream the
 * caller is using.
 * B, H or N equal to 0 is an empty problem: nothing is launched and 0 is returned,
 * whatever the pointers are (an empty torch tensor's data pointer is NULL).
 */
int tfgfa_fwd_bf16(const void* q, const void* k, const void* v, void* o, float* lse,
                   int B, int H, int N, int D, float softmax_scale, int causal,
                   void* hip_stream);

/*
 * The general forward: the surface of the reference's Triton wrapper
 * _flash_attn_forward(q, k, v, softmax_scale) (src/py/triton_implementation.py:184-197,
 * kernel :15-181): q (B, H, N_q, D), k and v (B, H, N_k, D), o like q, all strided
 * (4 element strides each, b/h/n/d, NULL = contiguous; rules as for
 * tfgfa_fwd_bf16_strided below), dtype
 * TFGFA_DTYPE_BF16 or TFGFA_DTYPE_F16, D any multiple of 8 from 8 to 128
 * (the Triton wrapper's d <= 128, :190), an explicit scale.  With causal == 1
 * the mask is top-left aligned as in the Triton kernel (:127): query i sees keys
 * j <= i and j < N_k.  N_k == 0 with N_q > 0 is TFGFA_ERR_BAD_SHAPE.  LSE, when
 * requested, is contiguous (B, H, N_q) float32.
 */
int tfgfa_fwd(const void* q, const int64_t* q_strides,
              const void* k, const int64_t* k_strides,
              const void* v, const int64_t* v_strides,
              void* o, const int64_t* o_strides, float* lse,
              int B, int H, int N_q, int N_k, int D, int dtype,
              float softmax_scale, int causal, void* hip_stream);

/*
 * The same attention over strided operands: each of q, k, v, o is described by
 * its base pointer and four element strides (batch, head, row, dim), as
 * torch's Tensor.stride() gives them; a NULL strides pointer means contiguous.
 * This lets a caller pass the (B, N, H, D) projections of a GPT-2 block as
 * (B, H, N, D) views (strides N*H*D, D, H*D, 1) and have O written straight
 * into a (B, N, H, D) buffer, so neither side needs a transposing copy
 * (the reference's caller views and transposes, src/py/model_inference.py:64-66,
 * copies Q, K, V with .contiguous(), :86-90, and O again, :92).
 * Rules (TFGFA_ERR_STRIDE otherwise): dim stride 1; batch, head and row strides
 * non-negative multiples of 8; row stride >= D; no two elements of O at one
 * address (checked: sorted by stride, each stride of a dimension of size > 1
 * exceeds the span of the smaller ones).  The stride of a dimension of size 1
 * is ignored.  (N + 128) * row stride * 2 must be < 2^31 (TFGFA_ERR_TOO_LARGE).
 * O must not overlap K or V (not checked).
 * LSE, when requested, stays a contiguous (B, H, N) float32 tensor.
 * No counterpart in the reference's C++ (its binding requires contiguous
 * tensors, torch_bind.cpp:14-16); it replaces the copies its caller makes.
 */
int tfgfa_fwd_bf16_strided(const void* q, const int64_t* q_strides,
                           const void* k, const int64_t* k_strides,
                           const void* v, const int64_t* v_strides,
                           void* o, const int64_t* o_strides, float* lse,
                           int B, int H, int N, int D, float softmax_scale, int causal,
                           void* hip_stream);

/*
 * One decode step over a KV cache: attention of one new query per (batch, head)
 * over the cached keys, bf16 in / bf16 out, fp32 softmax.
 *
 *   L_b = cache_seqlens[b] (+1 when appending), or N_max when cache_seqlens is NULL
 *   O[b,h,:]  = sum_{j < L_b} softmax_j(scale * q[b,h,:] . K[b,h,j,:]) * V[b,h,j,:]
 *   LSE[b,h]  = log sum_{j < L_b} exp(scale * q[b,h,:] . K[b,h,j,:])
 *
 * That is the last row of the causal forward over the first L_b tokens.  The
 * reference has no such step: its generate() re-runs the whole prefix through
 * the model for every new token (src/py/model_inference.py:199-228, timed at
 * :444-457), computing this row as part of a full causal forward.
 *
 * Operands (element strides, last dimension dense, other strides non-negative
 * multiples of 8, as Tensor.stride() gives them):
 *   q, o              (B, H, 64)        strides [b, h, d]
 *   k_cache, v_cache  (B, H, N_max, 64) strides [b, h, n, d], n >= 64
 *   k_new, v_new      (B, H, 64)        strides [b, h, d]; both NULL or both set
 *   cache_seqlens     B int32 in device memory, valid cached rows per batch row
 *   lse               (B, H) float32 contiguous, or NULL
 * With k_new/v_new set (requires cache_seqlens, else TFGFA_ERR_CACHE), row
 * L = cache_seqlens[b] of each cache receives k_new/v_new and attention covers
 * L + 1 keys; the caller advances cache_seqlens afterwards.  L_b = 0 gives
 * O = 0 and LSE = -inf.  A length that does not fit (cache_seqlens[b] < 0 or
 * cache_seqlens[b] + append > N_max) is only visible on the device: that batch
 * row gets NaN in O and LSE, and nothing is appended or attended for it.
 * Cache rows at or past the length never reach the result, but the first rows
 * of a chunk may be loaded (within the N_max rows of the cache) before the
 * length is known.
 *
 * workspace: device memory for split-sequence work (16-byte aligned), or NULL:
 * one arrival word per head (B*H*128 bytes rounded up to 256), then the
 * partials (B*H*260 bytes per split).  When B*H leaves most CUs idle, the cache
 * sequence is split over up to (workspace_bytes - arrival bytes) / (B*H*260)
 * workgroups per head, and the workgroup that finishes last merges the head's
 * partials (one kernel per step); with NULL (or too small for two splits) each
 * head is one workgroup, correct but slower for small B*H.  The workspace needs
 * no initialisation (every call leaves its arrival words at zero and installs
 * its own random tag over whatever they hold).  Calls sharing a workspace must
 * be ordered on one stream.
 */
int tfgfa_decode_bf16(const void* q, const int64_t* q_strides,
                      void* k_cache, const int64_t* k_strides,
                      void* v_cache, const int64_t* v_strides,
                      const void* k_new, const int64_t* k_new_strides,
                      const void* v_new, const int64_t* v_new_strides,
                      const int* cache_seqlens,
                      void* o, const int64_t* o_strides, float* lse,
                      int B, int H, int N_max, int D, float softmax_scale,
                      void* workspace, size_t workspace_bytes, void* hip_stream);

/*
 * Workspace bytes that let tfgfa_decode_bf16 use every split it may choose
 * for these sizes (0 when B, H or N_max is not positive).  Independent of the
 * device.  No counterpart in the reference.
 */
size_t tfgfa_decode_workspace_bytes(int B, int H, int N_max);

/*
 * tfgfa_decode_bf16 widened to the element types and head dims of tfgfa_fwd:
 * dtype TFGFA_DTYPE_BF16 or TFGFA_DTYPE_F16 for q, the caches, k_new, v_new and
 * o (fp32 softmax either way), D a multiple of 8 in [8, 128] (the cache row
 * stride n >= D).  Everything else - operands, lengths, append, NaN for
 * invalid lengths, workspace - as tfgfa_decode_bf16, with partials of
 * B*H*(D+1)*4 bytes per split after the arrival words.  With dtype TFGFA_DTYPE_BF16 and D = 64 the results are
 * bitwise those of tfgfa_decode_bf16.  Replaces, as tfgfa_decode_bf16 does,
 * the per-token full forward of generate() (src/py/model_inference.py:199-228),
 * for the fp16 / d <= 128 surface of the Triton wrapper
 * (src/py/triton_implementation.py:184-197).
 */
int tfgfa_decode(const void* q, const int64_t* q_strides,
                 void* k_cache, const int64_t* k_strides,
                 void* v_cache, const int64_t* v_strides,
                 const void* k_new, const int64_t* k_new_strides,
                 const void* v_new, const int64_t* v_new_strides,
                 const int* cache_seqlens,
                 void* o, const int64_t* o_strides, float* lse,
                 int B, int H, int N_max, int D, int dtype, float softmax_scale,
                 void* workspace, size_t workspace_bytes, void* hip_stream);

/*
 * Workspace bytes that let tfgfa_decode use every split it may choose for head
 * dim D (0 when B, H or N_max is not positive or D is not a multiple of 8 in
 * [8, 128]).  tfgfa_decode_workspace_bytes(B, H, N_max) equals this with
 * D = 64.  No counterpart in the reference.
 */
size_t tfgfa_decode_workspace_size(int B, int H, int N_max, int D);

/*
 * The split tfgfa_decode chooses: the number of workgroups S each head's cache is divided
 * over (1: one workgroup per head, no workspace used) on a device of cu_count CUs with a
 * workspace of workspace_bytes (0: none).  A workspace of exactly
 *   (B*H*128 rounded up to 256) + B*H*S*(D+1)*4 bytes
 * runs the same split.  0 when a size is out of range.  Host arithmetic only (no HIP call).
 * No counterpart in the reference: for callers sizing a workspace exactly.
 */
int tfgfa_decode_splits(int B, int H, int N_max, int D, int cu_count, size_t workspace_bytes);

/*
 * Bytes of tfgfa_decode_noalloc's static scratch (320 KiB).  No counterpart in the reference.
 */
size_t tfgfa_decode_scratch_bytes(void);

/*
 * tfgfa_decode without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  Operands, results and errors as tfgfa_decode; the arrival
 * words and split partials go to a static 320 KiB scratch array of the library instead (one
 * per GPU, held until the process ends), and the call allocates nothing.  The scratch acts
 * as a 320 KiB workspace: results are bitwise those of tfgfa_decode with a workspace of
 * tfgfa_decode_scratch_bytes() bytes, and so with any workspace that holds the library's
 * split (arrival words plus B*H*S*(D+1)*4 bytes), which 320 KiB does on a 256-CU MI355X
 * for every shape (at most 280 KiB).  On a part where the split would not fit, the call
 * splits only as far as the scratch holds (correct, a different split).  The first call on
 * a device looks the scratch up (hipGetSymbolAddress), also when that call is made during
 * stream capture.  Every call on one GPU shares that
 * GPU's scratch (it keeps the last call's partials, and its arrival words end at zero):
 * calls that overlap on one GPU, e.g. on two streams at once, race and must be ordered by
 * the caller.
 */
int tfgfa_decode_noalloc(const void* q, const int64_t* q_strides,
                         void* k_cache, const int64_t* k_strides,
                         void* v_cache, const int64_t* v_strides,
                         const void* k_new, const int64_t* k_new_strides,
                         const void* v_new, const int64_t* v_new_strides,
                         const int* cache_seqlens,
                         void* o, const int64_t* o_strides, float* lse,
                         int B, int H, int N_max, int D, int dtype, float softmax_scale,
                         void* hip_stream);

/*
 * A plain streaming read of `bytes` bytes at device pointer p (16-byte aligned, a multiple of
 * 16 bytes), writing meaningless words into `sink` (4096 uint32, device memory): the floor a
 * decode step's cache reads are measured against (bench.py's decode_split legs).  No counterpart
 * in the reference; measurement only.
 */
int tfgfa_stream_read(const void* p, size_t bytes, void* sink, void* hip_stream);

/*
 * Human-readable text for a status code returned by any tfgfa_* function.
 * The string is static.  Replaces the TORCH_CHECK messages of
 * src/cpp/torch_bind.cpp:13-19, :41 for errors detected below the binding
 * (the reference drops launcher errors, torch_bind.cpp:34-39).
 */
const char* tfgfa_strerror(int status);

/*
 * Properties of the current HIP device, queried once per device and cached
 * (the reference queries device 0 on every call, v1.cu:7-8).  Any output
 * pointer may be NULL.  `arch` receives the gcnArchName (e.g. "gfx950:sramecc+:xnack-").
 */
int tfgfa_device_info(int* cu_count, int* sclk_mhz, char* arch, int arch_len);

/* ABI version of the loaded library (TFGFA_ABI_VERSION at build time). */
int tfgfa_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* TFGFA_H */
