// The reference module's other operators, for gfx950: a device copy, FP32 attention
// scores, an FP32 attention forward, and a 16x64x16 FP16 matrix product on MFMA.
// They are off the hot path (correctness and a drop-in module surface matter, not
// peak speed), so the kernels are plain: FP32 SIMT tiles staged through LDS, and
// one wavefront per 16x16 product. Every kernel reads with element-sized loads, so
// any pointer aligned to its element type works (views with offsets included).
//
// Entry points (include/fa2_mi355x.h):
//   fa2_copy                    <- copy_cuda (reference csrc/copy_kernel.cu:23-53)
//   fa2_attention_scores_f32    <- naive_attention_scores (csrc/naive_attention.cu:174-201, 330-418)
//   fa2_attention_forward_f32   <- naive_attention_forward, block_attention_forward
//                                  (csrc/naive_attention.cu:48-172, 249-328, 420-502),
//                                  tiled_attention_forward (csrc/tiled_attention.cu:273-333),
//                                  tilewise_attention_forward (csrc/tilewise_attention.cu:337-388)
//   fa2_matmul_16x64x16_f16     <- wmma_matmul_16x64x16 (csrc/wmma_matmul.cu:51-193, 250-315)

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#include "fa2_mi355x.h"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

int hip_status(hipError_t err) {
    return err == hipSuccess ? FA2_STATUS_SUCCESS : FA2_STATUS_HIP_ERROR_BASE + (int)err;
}

bool aligned_to(const void* p, uintptr_t bytes) {
    return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0;
}

// ---------------------------------------------------------------------------
// Copy: grid-stride over elements of the widest size (16, 8, 4, 2 or 1 bytes)
// that divides both addresses and the byte count.
template <typename T>
__global__ __launch_bounds__(256) void copy_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                   int64_t count) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride)
        dst[i] = src[i];
}

template <typename T>
hipError_t launch_copy(const void* src, void* dst, int64_t bytes, hipStream_t stream) {
    const int64_t count = bytes / (int64_t)sizeof(T);
    const int64_t blocks = count / 256 + (count % 256 != 0);
    const unsigned grid = (unsigned)(blocks < 65536 ? blocks : 65536);
    hipLaunchKernelGGL((copy_kernel<T>), dim3(grid), dim3(256), 0, stream, static_cast<const T*>(src),
                       static_cast<T*>(dst), count);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Scores S[bh][i][j] = scale * sum_d Q[bh][i][d] K[bh][j][d], FP32. A workgroup
// (16 x 16 threads) computes a 64 x 64 block of S; thread (tx, ty) owns rows
// ty + 16a and columns tx + 16b (a, b < 4). Q and K rows are staged through LDS
// 16 dimensions at a time, transposed ([d][row]) so the inner loop reads rows
// across lanes without bank conflicts. Sums run over d in order with FMAs.
constexpr int kScoreTile = 64;
constexpr int kScoreChunk = 16;

__global__ __launch_bounds__(256) void scores_f32_kernel(const float* __restrict__ query,
                                                         const float* __restrict__ key,
                                                         float* __restrict__ scores, int seq_len,
                                                         int head_dim, int tiles, float scale) {
    __shared__ float q_s[kScoreChunk][kScoreTile + 1];
    __shared__ float k_s[kScoreChunk][kScoreTile + 1];
    const int tx = threadIdx.x & 15;
    const int ty = threadIdx.x >> 4;
    const int64_t block = blockIdx.x;
    const int64_t bh = block / ((int64_t)tiles * tiles);
    const int rem = (int)(block - bh * tiles * tiles);
    const int row0 = (rem / tiles) * kScoreTile;
    const int col0 = (rem % tiles) * kScoreTile;
    const float* q_head = query + bh * seq_len * (int64_t)head_dim;
    const float* k_head = key + bh * seq_len * (int64_t)head_dim;

    float acc[4][4] = {};
    for (int d0 = 0; d0 < head_dim; d0 += kScoreChunk) {
        // 64 rows x 16 dims of Q and of K: four elements of each per thread;
        // consecutive threads read consecutive dimensions of one row.
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int idx = threadIdx.x + 256 * e;
            const int r = idx >> 4, dd = idx & 15;
            const int d = d0 + dd;
            const bool in_d = d < head_dim;
            q_s[dd][r] = (in_d && row0 + r < seq_len) ? q_head[(int64_t)(row0 + r) * head_dim + d] : 0.0f;
            k_s[dd][r] = (in_d && col0 + r < seq_len) ? k_head[(int64_t)(col0 + r) * head_dim + d] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int dd = 0; dd < kScoreChunk; ++dd) {
            float qa[4], kb[4];
#pragma unroll
            for (int a = 0; a < 4; ++a) qa[a] = q_s[dd][ty + 16 * a];
#pragma unroll
            for (int b = 0; b < 4; ++b) kb[b] = k_s[dd][tx + 16 * b];
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int b = 0; b < 4; ++b) acc[a][b] = fmaf(qa[a], kb[b], acc[a][b]);
        }
        __syncthreads();
    }
    float* s_head = scores + bh * (int64_t)seq_len * seq_len;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        const int i = row0 + ty + 16 * a;
        if (i >= seq_len) continue;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int j = col0 + tx + 16 * b;
            if (j < seq_len) s_head[(int64_t)i * seq_len + j] = acc[a][b] * scale;
        }
    }
}

// ---------------------------------------------------------------------------
// FP32 attention forward (noncausal), head_dim kD = 64 or 128. A workgroup of 256
// threads owns 64 queries of one (batch, head); each query is handled by four
// consecutive lanes, each owning kD/4 dimensions of Q and of O. Keys stream in
// tiles of 32 rows of K and V through LDS. Per tile: partial dot products over
// the lane's dimensions, summed over the four lanes by two xor shuffles; the tile
// max updates the running max (online softmax, exp2 with log2(e) folded into the
// scale); O and l are rescaled once per tile. Keys past seq_len score -inf; lanes
// of queries past seq_len compute on a zero query and store nothing.
constexpr int kF32Queries = 64;
constexpr int kF32Keys = 32;

template <int kD>
__global__ __launch_bounds__(256) void attention_f32_kernel(const float* __restrict__ query,
                                                            const float* __restrict__ key,
                                                            const float* __restrict__ value,
                                                            float* __restrict__ output, int seq_len,
                                                            int query_tiles, float scale_log2) {
    constexpr int kPart = kD / 4;
    constexpr int kRow = kD + 4;  // LDS row stride (floats), keeps 16-byte alignment
    __shared__ __attribute__((aligned(16))) float k_s[kF32Keys][kRow];
    __shared__ __attribute__((aligned(16))) float v_s[kF32Keys][kRow];

    const int tid = threadIdx.x;
    const int64_t bh = blockIdx.x / query_tiles;
    const int tile = (int)(blockIdx.x - bh * query_tiles);
    const int q_index = tile * kF32Queries + (tid >> 2);
    const int d0 = (tid & 3) * kPart;
    const bool q_valid = q_index < seq_len;
    const int64_t head = bh * (int64_t)seq_len * kD;

    float q[kPart], acc[kPart];
#pragma unroll
    for (int i = 0; i < kPart; ++i) {
        q[i] = q_valid ? query[head + (int64_t)q_index * kD + d0 + i] : 0.0f;
        acc[i] = 0.0f;
    }
    float m_run = -INFINITY;  // running max of scaled (log2-domain) scores
    float l_run = 0.0f;

    for (int k0 = 0; k0 < seq_len; k0 += kF32Keys) {
        __syncthreads();  // the previous tile is consumed
        for (int e = tid; e < kF32Keys * kD; e += 256) {
            const int r = e / kD, c = e % kD;
            const bool in = k0 + r < seq_len;
            const int64_t src = head + (int64_t)(k0 + r) * kD + c;
            k_s[r][c] = in ? key[src] : 0.0f;
            v_s[r][c] = in ? value[src] : 0.0f;
        }
        __syncthreads();
        const int valid_keys = seq_len - k0 < kF32Keys ? seq_len - k0 : kF32Keys;

        float s[kF32Keys];
        float tile_max = -INFINITY;
#pragma unroll
        for (int j = 0; j < kF32Keys; ++j) {
            float partial = 0.0f;
#pragma unroll
            for (int i = 0; i < kPart; ++i) partial = fmaf(q[i], k_s[j][d0 + i], partial);
            partial += __shfl_xor(partial, 1);
            partial += __shfl_xor(partial, 2);
            s[j] = j < valid_keys ? partial * scale_log2 : -INFINITY;
            tile_max = fmaxf(tile_max, s[j]);
        }
        const float m_new = fmaxf(m_run, tile_max);  // finite: every tile has a valid key
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first tile
        l_run *= alpha;
#pragma unroll
        for (int i = 0; i < kPart; ++i) acc[i] *= alpha;
#pragma unroll
        for (int j = 0; j < kF32Keys; ++j) {
            const float p = __builtin_amdgcn_exp2f(s[j] - m_new);
            l_run += p;
#pragma unroll
            for (int i = 0; i < kPart; ++i) acc[i] = fmaf(p, v_s[j][d0 + i], acc[i]);
        }
        m_run = m_new;
    }
    if (!q_valid) return;
    const float inv_l = 1.0f / l_run;
#pragma unroll
    for (int i = 0; i < kPart; ++i) output[head + (int64_t)q_index * kD + d0 + i] = acc[i] * inv_l;
}

// ---------------------------------------------------------------------------
// C = A B for one 16x64 (A) by 64x16 (B) FP16 pair per wavefront, FP32 result, as
// two v_mfma_f32_16x16x32_f16. Operand layout of that instruction: lane l holds,
// for A, row l%16 and reduction indices 8(l/16)..8(l/16)+7; for B, column l%16
// and the same reduction indices; the 16x16 FP32 result gives lane l column l%16,
// rows 4(l/16)..4(l/16)+3.
__global__ __launch_bounds__(64) void matmul_16x64x16_kernel(const _Float16* __restrict__ a,
                                                             const _Float16* __restrict__ b,
                                                             float* __restrict__ c) {
    const int64_t m = blockIdx.x;
    const int lane = threadIdx.x;
    const int rc = lane & 15;       // row of A, column of B and of C
    const int kg = lane >> 4;       // reduction group
    const _Float16* a_m = a + m * 16 * 64;
    const _Float16* b_m = b + m * 64 * 16;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        f16x8 av, bv;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int k = 32 * h + 8 * kg + j;
            av[j] = a_m[rc * 64 + k];
            bv[j] = b_m[k * 16 + rc];
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc, 0, 0, 0);
    }
    float* c_m = c + m * 16 * 16;
#pragma unroll
    for (int i = 0; i < 4; ++i) c_m[(4 * kg + i) * 16 + rc] = acc[i];
}

}  // namespace

extern "C" int fa2_copy(const void* src, void* dst, int64_t bytes, void* stream) {
    if (bytes < 0) return FA2_STATUS_NEGATIVE_DIMENSION;
    if (bytes == 0) return FA2_STATUS_SUCCESS;
    if (!src || !dst) return FA2_STATUS_NULL_POINTER;
    const uintptr_t bits = reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) |
                           static_cast<uintptr_t>(bytes);
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t err;
    if ((bits & 15) == 0) err = launch_copy<u32x4>(src, dst, bytes, s);
    else if ((bits & 7) == 0) err = launch_copy<uint64_t>(src, dst, bytes, s);
    else if ((bits & 3) == 0) err = launch_copy<uint32_t>(src, dst, bytes, s);
    else if ((bits & 1) == 0) err = launch_copy<uint16_t>(src, dst, bytes, s);
    else err = launch_copy<uint8_t>(src, dst, bytes, s);
    return hip_status(err);
}

extern "C" int fa2_attention_scores_f32(const float* query, const float* key, float* scores,
                                        int64_t batch_heads, int64_t seq_len, int64_t head_dim,
                                        void* stream) {
    if (batch_heads < 0 || seq_len < 0 || head_dim < 0) return FA2_STATUS_NEGATIVE_DIMENSION;
    if (batch_heads == 0 || seq_len == 0) return FA2_STATUS_SUCCESS;
    if (!query || !key || !scores) return FA2_STATUS_NULL_POINTER;
    if (!aligned_to(query, 4) || !aligned_to(key, 4) || !aligned_to(scores, 4)) return FA2_STATUS_MISALIGNED;
    if (seq_len > INT32_MAX || head_dim > INT32_MAX) return FA2_STATUS_TOO_LARGE;
    const int64_t tiles = (seq_len + kScoreTile - 1) / kScoreTile;  // seq_len <= INT32_MAX: no overflow
    if (batch_heads > (int64_t)UINT32_MAX / (tiles * tiles)) return FA2_STATUS_TOO_LARGE;
    // scale = 1/sqrt(head_dim) in FP32, as the reference's host code computes it
    // (head_dim 0 gives +inf and scores of 0 * inf = NaN there too).
    const float scale = 1.0f / sqrtf((float)head_dim);
    hipLaunchKernelGGL(scores_f32_kernel, dim3((unsigned)(batch_heads * tiles * tiles)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), query, key, scores, (int)seq_len,
                       (int)head_dim, (int)tiles, scale);
    return hip_status(hipGetLastError());
}

extern "C" int fa2_attention_forward_f32(const float* query, const float* key, const float* value,
                                         float* output, int64_t batch_heads, int64_t seq_len,
                                         int64_t head_dim, void* stream) {
    if (batch_heads < 0 || seq_len < 0 || head_dim < 0) return FA2_STATUS_NEGATIVE_DIMENSION;
    if (head_dim != 64 && head_dim != 128) return FA2_STATUS_BAD_HEAD_DIM;
    if (batch_heads == 0 || seq_len == 0) return FA2_STATUS_SUCCESS;
    if (!query || !key || !value || !output) return FA2_STATUS_NULL_POINTER;
    if (!aligned_to(query, 4) || !aligned_to(key, 4) || !aligned_to(value, 4) || !aligned_to(output, 4))
        return FA2_STATUS_MISALIGNED;
    if (seq_len > INT32_MAX) return FA2_STATUS_TOO_LARGE;
    const int64_t tiles = (seq_len + kF32Queries - 1) / kF32Queries;  // seq_len <= INT32_MAX: no overflow
    if (batch_heads > (int64_t)UINT32_MAX / tiles) return FA2_STATUS_TOO_LARGE;
    const float scale_log2 = 1.0f / sqrtf((float)head_dim) * 1.4426950408889634074f;
    const dim3 grid((unsigned)(batch_heads * tiles));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (head_dim == 64)
        hipLaunchKernelGGL((attention_f32_kernel<64>), grid, dim3(256), 0, s, query, key, value, output,
                           (int)seq_len, (int)tiles, scale_log2);
    else
        hipLaunchKernelGGL((attention_f32_kernel<128>), grid, dim3(256), 0, s, query, key, value, output,
                           (int)seq_len, (int)tiles, scale_log2);
    return hip_status(hipGetLastError());
}

extern "C" int fa2_matmul_16x64x16_f16(const void* a, const void* b, float* c, int64_t batch,
                                       void* stream) {
    if (batch < 0) return FA2_STATUS_NEGATIVE_DIMENSION;
    if (batch == 0) return FA2_STATUS_SUCCESS;
    if (!a || !b || !c) return FA2_STATUS_NULL_POINTER;
    if (!aligned_to(a, 2) || !aligned_to(b, 2) || !aligned_to(c, 4)) return FA2_STATUS_MISALIGNED;
    if (batch > (int64_t)UINT32_MAX) return FA2_STATUS_TOO_LARGE;
    hipLaunchKernelGGL(matmul_16x64x16_kernel, dim3((unsigned)batch), dim3(64), 0,
                       static_cast<hipStream_t>(stream), static_cast<const _Float16*>(a),
                       static_cast<const _Float16*>(b), c);
    return hip_status(hipGetLastError());
}
