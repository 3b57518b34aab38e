/*
 * fa2_mi355x.h - C ABI of the MI355X (gfx950) FlashAttention-2 forward library.
 *
 * Library: flash_attention_2_lab_amd/libfa2_mi355x.so (hand-written HIP for gfx950).
 *
 * Every entry point takes plain device pointers and sizes; no torch or HIP types
 * appear in the signatures. The attention tensors are row-major
 * [batch, heads, seq_len, head_dim] and contiguous: FP16 (IEEE binary16) and
 * 16-byte aligned for the tensor-core entries, FP32 and 4-byte aligned for the
 * FP32 entries. Output buffers are written, never read; inputs are read-only and
 * must not overlap the output. Calls are asynchronous:
 * the kernel is enqueued on `stream` (a hipStream_t passed as void*; NULL means
 * the legacy default stream) and no host synchronisation happens. The kernel runs
 * on the calling thread's current HIP device (hipSetDevice); the pointers and the
 * stream must belong to that device. The entries allocate nothing and issue no
 * memset, so they may be recorded into a HIP graph.
 *
 * Status codes: 0 on success; a positive FA2_STATUS_* value for an argument the
 * library rejects before touching the GPU; FA2_STATUS_HIP_ERROR_BASE + hipError_t
 * when the HIP runtime reports a launch error. fa2_status_string() names each.
 */
#ifndef FA2_MI355X_H
#define FA2_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA2_MI355X_ABI_VERSION 8

enum fa2_status {
    FA2_STATUS_SUCCESS = 0,
    FA2_STATUS_NULL_POINTER = 1,        /* non-empty problem with a NULL tensor pointer      */
    FA2_STATUS_NEGATIVE_DIMENSION = 2,  /* batch, heads, seq_len or head_dim below zero      */
    FA2_STATUS_BAD_HEAD_DIM = 3,        /* head_dim not supported by the entry               */
    FA2_STATUS_BAD_SEQUENCE_LENGTH = 4, /* seq_len not a multiple of the entry's key tile    */
    FA2_STATUS_MISALIGNED = 5,          /* a pointer below the entry's alignment             */
    FA2_STATUS_TOO_LARGE = 6,           /* seq_len > 2^24 or launch grid beyond 2^32 groups */
    FA2_STATUS_BAD_KEY_TILE = 7,        /* fa2_forward_tensorcore: key_tile not 16 or 32     */
    FA2_STATUS_BAD_KERNEL = 8,          /* fa2_forward_with_kernel: the kernel does not      */
                                        /* compute these sizes                               */
    FA2_STATUS_HIP_ERROR_BASE = 1000    /* + hipError_t from the launch                      */
};

/*
 * Fused attention forward, O = softmax(Q K^T / sqrt(64) [+ causal mask]) V.
 * FP16 in/out, FP32 accumulation and FP32 online softmax; P is rounded to FP16
 * before the P.V product. The softmax denominator differs from the reference's FP32
 * sum of unrounded probabilities in most kernels: they add the FP16-rounded P in
 * pairs (an FP16 add) and accumulate the pair sums into FP32 with v_dot2, so that
 * O is a convex combination of the P the product used. The causal kernel for 512
 * to 2047 keys on few heads (FA2_KERNEL_KEY_SPLIT_PAIRS16) sums unrounded FP32 P.
 * Outputs stay within atol 2e-3 + rtol 1e-2 of the FP32 formula.
 * NaN and +-inf inputs make NaN or inf exactly the outputs the FP32 formula does,
 * except that a causal row i < j may or may not see a NaN or inf in value row j,
 * where the formula's 0 * NaN always does.
 * causal != 0 masks key j > query i.
 *
 * Replaces tensorcore_attention_forward_production_128x128
 *   (reference csrc/tensorcore_attention.cu:3191-3203, implementation 2969-3123,
 *    validation 2731-2823; binding csrc/bindings.cpp:63-68 and 136-140).
 * Preconditions mirror the reference: head_dim == 64, seq_len % 128 == 0.
 * batch, heads or seq_len == 0 returns FA2_STATUS_SUCCESS without a launch
 * (reference csrc/tensorcore_attention.cu:3003-3009).
 */
int fa2_forward_production_128x128(const void* query, const void* key, const void* value,
                                   void* output, int64_t batch, int64_t heads,
                                   int64_t seq_len, int64_t head_dim, int causal,
                                   void* stream);

/*
 * Noncausal fused attention forward for any seq_len that is a multiple of
 * key_tile (16 or 32); the last query block and key tile may be partial. Same
 * arithmetic and output contract as fa2_forward_production_128x128.
 *
 * Replaces the reference's Bc=16/Bc=32 tensor-core entry points, which differ
 * only in the sequence-length divisor they accept:
 *   tensorcore_attention_forward                    key_tile 16
 *   tensorcore_attention_forward_bc32               key_tile 32
 *   tensorcore_attention_forward_bc32_raw_pv        key_tile 32
 *   tensorcore_attention_forward_bc32_raw_qk_raw_pv key_tile 32
 *   (reference csrc/tensorcore_attention.cu:3131-3189, implementation 2826-2967,
 *    validation 2731-2823; bindings csrc/bindings.cpp:39-61 and 113-134).
 */
int fa2_forward_tensorcore(const void* query, const void* key, const void* value,
                           void* output, int64_t batch, int64_t heads, int64_t seq_len,
                           int64_t head_dim, int64_t key_tile, void* stream);

/*
 * Device-to-device copy of `bytes` bytes (src and dst must not overlap).
 * Replaces copy_cuda (reference csrc/copy_kernel.cu:23-53; binding
 * csrc/bindings.cpp:71-75), which copies a contiguous floating-point tensor.
 */
int fa2_copy(const void* src, void* dst, int64_t bytes, void* stream);

/*
 * FP32 attention scores S = Q K^T / sqrt(head_dim) for each of batch_heads
 * [seq_len, head_dim] slabs of Q and K; writes S as [batch_heads, seq_len, seq_len].
 * Replaces naive_attention_scores (reference csrc/naive_attention.cu:174-201,
 * 330-418; binding csrc/bindings.cpp:83-87).
 */
int fa2_attention_scores_f32(const float* query, const float* key, float* scores,
                             int64_t batch_heads, int64_t seq_len, int64_t head_dim,
                             void* stream);

/*
 * FP32 attention forward, noncausal, O = softmax(Q K^T / sqrt(head_dim)) V, for
 * head_dim 64 or 128 and any seq_len. Replaces the reference's four FP32 SIMT
 * forwards, which compute the same attention with different thread mappings:
 *   naive_attention_forward     (reference csrc/naive_attention.cu:112-172, 249-328)
 *   block_attention_forward     (csrc/naive_attention.cu:48-110, 420-502)
 *   tiled_attention_forward     (csrc/tiled_attention.cu:273-333), head_dim 64
 *   tilewise_attention_forward  (csrc/tilewise_attention.cu:337-388), head_dim 64
 *   (bindings csrc/bindings.cpp:77-81, 89-105).
 */
int fa2_attention_forward_f32(const float* query, const float* key, const float* value,
                              float* output, int64_t batch_heads, int64_t seq_len,
                              int64_t head_dim, void* stream);

/*
 * C[i] = A[i] B[i] for `batch` pairs of a 16x64 and a 64x16 FP16 matrix (row-major,
 * contiguous), FP32 result [batch, 16, 16]; two v_mfma_f32_16x16x32_f16 per pair.
 * Replaces wmma_matmul_16x64x16 (reference csrc/wmma_matmul.cu:51-193, 250-315;
 * binding csrc/bindings.cpp:107-111).
 */
int fa2_matmul_16x64x16_f16(const void* a, const void* b, float* c, int64_t batch, void* stream);

/* Human-readable name of a status code returned by this library (static storage). */
const char* fa2_status_string(int status);

/* FA2_MI355X_ABI_VERSION of the loaded library. */
int fa2_abi_version(void);

/* Kernels of the FP16 forward entries (fa2_forward_plan). */
enum fa2_forward_kernel {
    FA2_KERNEL_NONE = 0,             /* empty or rejected sizes: nothing is launched       */
    FA2_KERNEL_256_QUERY = 1,        /* 256 queries per workgroup, one query tile each     */
    FA2_KERNEL_256_QUERY_PAIRS = 2,  /* 256 queries per workgroup, causal tiles T-1-p, p   */
    FA2_KERNEL_128_QUERY = 3,        /* 128 queries per workgroup                          */
    FA2_KERNEL_KEY_SPLIT_64 = 4,     /* 32 queries per workgroup, keys split over 4 waves, */
                                     /* 64-key tiles                                       */
    FA2_KERNEL_KEY_SPLIT_32 = 5,     /* the same with 32-key tiles                         */
    FA2_KERNEL_KEY_SPLIT_8_WAVES = 6, /* keys split over 8 waves, 32-key tiles             */
    FA2_KERNEL_KEY_SPLIT_PAIRS16 = 7, /* causal: 16-query blocks p and N/16-1-p of a head  */
                                      /* per workgroup, keys split over 4 waves            */
    FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES = 8, /* as KEY_SPLIT_64, plus 4 waves that only fetch */
                                           /* K/V tiles into LDS for the 4 computing waves  */
    FA2_KERNEL_128_QUERY_SPLIT_PAIRS = 9   /* causal: 128-query tiles T-1-p and p of a head */
                                           /* per 8-wave workgroup, keys split between two  */
                                           /* groups of 4 waves                             */
};

/*
 * The kernel fa2_forward_production_128x128 and fa2_forward_tensorcore launch for
 * these sizes (head_dim 64, any accepted seq_len; causal for the production entry
 * only), or FA2_KERNEL_NONE when they launch nothing. No GPU work, no HIP call.
 * No counterpart in the reference (whose production entry has one kernel): it is
 * for callers and tests that need to know which schedule a shape gets.
 */
int fa2_forward_plan(int64_t batch, int64_t heads, int64_t seq_len, int causal);

/*
 * fa2_forward_production_128x128 run on a chosen kernel instead of the one
 * fa2_forward_plan names: the same checks, arithmetic and output contract, then
 * FA2_STATUS_BAD_KERNEL unless `kernel` computes these sizes:
 *   FA2_KERNEL_256_QUERY               seq_len % 256 == 0
 *   FA2_KERNEL_256_QUERY_PAIRS         causal, seq_len % 512 == 0
 *   FA2_KERNEL_128_QUERY               any (seq_len % 128 == 0)
 *   FA2_KERNEL_128_QUERY_SPLIT_PAIRS   causal, seq_len % 256 == 0, seq_len >= 1024
 *   FA2_KERNEL_KEY_SPLIT_64, _32, _8_WAVES   any
 *   FA2_KERNEL_KEY_SPLIT_PAIRS16       causal, seq_len % 64 == 0, seq_len >= 512
 *   FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES  noncausal
 * No counterpart in the reference (whose production entry has one kernel): it is for
 * re-measuring the kernel choice - timing the kernels on either side of each routing
 * threshold - and for tests that hold every kernel to the oracle on shapes it is not
 * routed to.
 */
int fa2_forward_with_kernel(int kernel, const void* query, const void* key, const void* value,
                            void* output, int64_t batch, int64_t heads, int64_t seq_len,
                            int64_t head_dim, int causal, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FA2_MI355X_H */
