// FlashAttention-2 forward, FP16 in/out, head_dim 64, for AMD Instinct MI355X (gfx950).
//
// Computes O = softmax(Q K^T * scale [+ causal mask]) V per (batch, head) with FP32
// accumulation, as the reference's production kernel does
// (reference csrc/tensorcore_attention.cu:2019-2727). The algorithm is the same
// FA2 streaming softmax; the mapping onto the hardware is CDNA4-specific:
//
//  * One wavefront (64 lanes) owns 32 queries. Scores are produced transposed,
//    S^T[key][query] = K * Q^T, with v_mfma_f32_32x32x16_f16: in the 32x32 FP32
//    accumulator layout a lane holds one column (= one query) and 16 rows (keys),
//    so the per-query max and sum are in-lane reductions plus one
//    v_permlane32_swap between lane l and lane l^32.
//  * The MFMA row r of a 32-key block is fed from key sigma(r) = r with bits 2 and 3
//    swapped. With that permutation the 8 FP32 scores a lane holds for C-registers
//    8t..8t+7 are exactly 8 consecutive keys, so P^T can be converted to FP16 in
//    registers and used directly as the B operand of O^T += V^T P^T.
//  * V^T operands come from the row-major V tile in LDS through ds_read_b64_tr_b16
//    (LDS transpose read), so K and V are staged identically.
//  * O^T lives in the MFMA accumulators: every accumulator of a lane belongs to the
//    lane's own query, so the online-softmax rescale needs no cross-lane traffic.
//  * K/V tiles (64 keys x 64 dims, 8 KiB each) are double-buffered in LDS with a
//    16-byte-chunk XOR swizzle that keeps both the K reads (ds_read_b128) and the
//    V transpose reads free of bank conflicts; tile j+1 is prefetched into
//    registers while tile j is computed, one barrier per tile.
//  * Causal mode stops the key loop at the diagonal, skips tiles a wave can never
//    see and masks only diagonal tiles (key > query -> -inf).
//  * Workgroup ids are remapped so all query tiles of one (batch, head) land on the
//    same XCD (dispatch is round-robin over the 8 XCDs), keeping that head's K/V
//    resident in one L2; causal tiles run heaviest first.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#include "fa2_mi355x.h"

namespace {

constexpr int kHeadDim = 64;
constexpr int kQueriesPerWave = 32;
constexpr int kKeysPerTile = 64;                          // BN
constexpr int kRowBytes = kHeadDim * 2;                   // 128 B per key row
constexpr int kChunksPerTile = kKeysPerTile * kRowBytes / 16;  // 512 chunks of 16 B
constexpr int kTileBytes = kKeysPerTile * kRowBytes;      // 8 KiB
constexpr int kQueryTileAlign = 128;                      // reference kProductionBlockM/N

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __fp16 fp16x4_lds __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define FA2_LDS __attribute__((address_space(3)))

// XOR applied to the 16-byte chunk index of key row `row` inside an LDS tile.
// Bits: chunk ^= ((row & 3) << 1) | ((row >> 3) & 1).
//  - K reads (A operand of K*Q^T): 8 consecutive lanes read rows sigma(8g..8g+7),
//    whose bits {0,1,3} take all 8 values -> 8 distinct chunks, 128 B, no conflict.
//  - V transpose reads: a 16-lane group reads rows 4a..4a+3 at one 32-byte
//    column pair; (row & 3) << 1 moves each row to a different pair.
__device__ __forceinline__ int tile_swizzle(int row) {
    return ((row & 3) << 1) | ((row >> 3) & 1);
}

// MFMA row r of a 32-key block reads key sigma(r): bits 2 and 3 of r swapped.
__device__ __forceinline__ int key_of_mfma_row(int r) {
    return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);
}

__device__ __forceinline__ float max_across_halves(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float sum_across_halves(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ f16x2 pack_rn(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_convertvector(v, f16x2);  // v_cvt_pk_f16_f32, round to nearest even
}

__device__ __forceinline__ f16x4 lds_read_transposed(const uint8_t* p) {
    const fp16x4_lds r = __builtin_amdgcn_ds_read_tr16_b64_v4f16((FA2_LDS fp16x4_lds*)(p));
    return __builtin_bit_cast(f16x4, r);
}

// Registers that carry one 64x64 FP16 tile from global memory to LDS.
template <int kThreads>
struct TileCarrier {
    static constexpr int kPerThread = kChunksPerTile / kThreads;
    static_assert(kChunksPerTile % kThreads == 0, "tile chunks must split evenly");
    u32x4 r[kPerThread];

    __device__ __forceinline__ void load(const uint8_t* __restrict__ src, int tid) {
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int c = tid + i * kThreads;
            r[i] = *reinterpret_cast<const u32x4*>(src + (c >> 3) * kRowBytes + (c & 7) * 16);
        }
    }

    __device__ __forceinline__ void store(uint8_t* dst, int tid) const {
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int c = tid + i * kThreads;
            const int row = c >> 3;
            *reinterpret_cast<u32x4*>(dst + row * kRowBytes + (((c & 7) ^ tile_swizzle(row)) << 4)) =
                r[i];
        }
    }
};

template <bool kCausal, int kWaves>
__global__ __launch_bounds__(kWaves * 64)
void fa2_forward_d64_kernel(const _Float16* __restrict__ query,
                            const _Float16* __restrict__ key,
                            const _Float16* __restrict__ value,
                            _Float16* __restrict__ output,
                            int seq_len, int num_query_tiles, float scale_log2) {
    constexpr int kThreads = kWaves * 64;
    constexpr int kBlockM = kWaves * kQueriesPerWave;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2][2][kTileBytes];  // [buffer][K|V]

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int lq = lane & 31;   // query column owned by this lane
    const int half = lane >> 5; // which 16 of each 32 keys this lane holds

    // Workgroup -> (batch*head, query tile). Dispatch is round-robin over 8 XCDs
    // (id % 8); give every XCD a contiguous range of logical tiles so the query
    // tiles of one head share that XCD's L2.
    const uint32_t groups = gridDim.x;
    const uint32_t xcd = blockIdx.x & 7u;
    const uint32_t slot = blockIdx.x >> 3;
    const uint32_t per_xcd = groups >> 3;
    const uint32_t extra = groups & 7u;
    const uint32_t logical = xcd * per_xcd + min(xcd, extra) + slot;
    const uint32_t bh = logical / (uint32_t)num_query_tiles;
    uint32_t qtile = logical - bh * (uint32_t)num_query_tiles;
    if (kCausal) qtile = (uint32_t)num_query_tiles - 1u - qtile;  // heaviest tiles first

    const size_t head_offset = (size_t)bh * (size_t)seq_len * kHeadDim;
    const _Float16* __restrict__ q_head = query + head_offset;
    const uint8_t* __restrict__ k_head = reinterpret_cast<const uint8_t*>(key + head_offset);
    const uint8_t* __restrict__ v_head = reinterpret_cast<const uint8_t*>(value + head_offset);
    _Float16* __restrict__ o_head = output + head_offset;

    const int q_block = (int)qtile * kBlockM;
    const int q_wave = q_block + wave * kQueriesPerWave;
    const int my_query = q_wave + lq;

    // Q^T as the B operand of K*Q^T: lane holds dims 16ks + 8*half + 0..7 of its query.
    f16x8 q_frag[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
        q_frag[ks] = *reinterpret_cast<const f16x8*>(q_head + (size_t)my_query * kHeadDim +
                                                      ks * 16 + half * 8);

    const int num_tiles = kCausal ? (q_block + kBlockM - 1) / kKeysPerTile + 1
                                  : seq_len / kKeysPerTile;

    // Per-lane LDS byte offsets.
    // K (A operand): MFMA row lq -> key row sigma(lq) (+32 for block 1), chunk 2ks + half.
    const int k_row = key_of_mfma_row(lq);
    const int k_swz = tile_swizzle(k_row);
    int k_off[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) k_off[ks] = k_row * kRowBytes + (((2 * ks + half) ^ k_swz) << 4);
    // V^T (A operand) through transpose reads. In a 16-lane group g, lane i reads 4
    // halves at key row base + i/4, dims d0 + 4*(i%4); the read returns, to lane i,
    // dim d0 + i at keys base..base+3. Row base = 32b + 16t + 8*half + 4r.
    const int grp = lane >> 4;
    const int i16 = lane & 15;
    const int v_row = 8 * half + (i16 >> 2);
    const int v_swz = ((i16 >> 2) << 1) | half;  // tile_swizzle(v_row + 32b + 16t + 4r)
    int v_off[2];
#pragma unroll
    for (int dblk = 0; dblk < 2; ++dblk) {
        const int chunk = 4 * dblk + 2 * (grp & 1) + ((i16 & 3) >> 1);
        v_off[dblk] = v_row * kRowBytes + ((chunk ^ v_swz) << 4) + 8 * (i16 & 1);
    }

    f32x16 o_acc[2];
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
        for (int i = 0; i < 16; ++i) o_acc[d][i] = 0.0f;
    float m_run = -INFINITY;  // running max of raw scores (unscaled) for my_query
    float l_run = 0.0f;       // this lane's share of the running softmax denominator

    TileCarrier<kThreads> k_carry, v_carry;
    k_carry.load(k_head, tid);
    v_carry.load(v_head, tid);
    k_carry.store(&smem[0][0][0], tid);
    v_carry.store(&smem[0][1][0], tid);
    __syncthreads();

    for (int j = 0; j < num_tiles; ++j) {
        const int buf = j & 1;
        const bool has_next = j + 1 < num_tiles;
        if (has_next) {
            k_carry.load(k_head + (size_t)(j + 1) * kTileBytes, tid);
            v_carry.load(v_head + (size_t)(j + 1) * kTileBytes, tid);
        }
        const int k0 = j * kKeysPerTile;
        // Causal: a wave whose last query precedes the tile sees none of it.
        const bool active = !kCausal || k0 <= q_wave + kQueriesPerWave - 1;
        if (active) {
            const uint8_t* k_lds = &smem[buf][0][0];
            const uint8_t* v_lds = &smem[buf][1][0];

            // S^T = K Q^T for two 32-key blocks.
            f32x16 s[2];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
#pragma unroll
                for (int i = 0; i < 16; ++i) s[b][i] = 0.0f;
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const f16x8 kf = *reinterpret_cast<const f16x8*>(k_lds + b * 32 * kRowBytes + k_off[ks]);
                    s[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, q_frag[ks], s[b], 0, 0, 0);
                }
            }

            // Accumulator register i of block b holds key k0 + 32b + 16(i/8) + 8*half + i%8.
            if (kCausal && k0 + kKeysPerTile - 1 > q_wave) {
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int key_index = k0 + 32 * b + 16 * (i >> 3) + 8 * half + (i & 7);
                        if (key_index > my_query) s[b][i] = -INFINITY;
                    }
            }

            float tile_max = -INFINITY;
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int i = 0; i < 16; i += 2) tile_max = fmaxf(tile_max, fmaxf(s[b][i], s[b][i + 1]));
            tile_max = max_across_halves(tile_max);
            const float m_new = fmaxf(m_run, tile_max);
            // m_run == -inf only before the first tile, where the correction is 0.
            const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * scale_log2);
            const float m_scaled = m_new * scale_log2;

            // p = exp(scale * (s - m)) = 2^(s * scale*log2e - m * scale*log2e).
            float p_sum = 0.0f;
            f16x8 p_frag[2][2];
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    float p[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        p[e] = __builtin_amdgcn_exp2f(fmaf(s[b][8 * t + e], scale_log2, -m_scaled));
                        p_sum += p[e];
                    }
                    const f16x2 p01 = pack_rn(p[0], p[1]);
                    const f16x2 p23 = pack_rn(p[2], p[3]);
                    const f16x2 p45 = pack_rn(p[4], p[5]);
                    const f16x2 p67 = pack_rn(p[6], p[7]);
                    const f16x4 lo = __builtin_shufflevector(p01, p23, 0, 1, 2, 3);
                    const f16x4 hi = __builtin_shufflevector(p45, p67, 0, 1, 2, 3);
                    p_frag[b][t] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                }
            l_run = l_run * alpha + p_sum;
            m_run = m_new;
#pragma unroll
            for (int d = 0; d < 2; ++d)
#pragma unroll
                for (int i = 0; i < 16; ++i) o_acc[d][i] *= alpha;

            // O^T += V^T P^T, 16 keys per MFMA.
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const int row_base = (32 * b + 16 * t) * kRowBytes;
#pragma unroll
                    for (int dblk = 0; dblk < 2; ++dblk) {
                        const f16x4 v_lo = lds_read_transposed(v_lds + row_base + v_off[dblk]);
                        const f16x4 v_hi = lds_read_transposed(v_lds + row_base + 4 * kRowBytes + v_off[dblk]);
                        const f16x8 vf = __builtin_shufflevector(v_lo, v_hi, 0, 1, 2, 3, 4, 5, 6, 7);
                        o_acc[dblk] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, p_frag[b][t], o_acc[dblk], 0, 0, 0);
                    }
                }
        }
        if (has_next) {
            k_carry.store(&smem[buf ^ 1][0][0], tid);
            v_carry.store(&smem[buf ^ 1][1][0], tid);
        }
        __syncthreads();
    }

    // Epilogue: O = O^T / l. Accumulator i of d-block dblk holds dim
    // 32*dblk + 8*(i/4) + 4*half + i%4 of my_query.
    const float inv_l = 1.0f / sum_across_halves(l_run);
    _Float16* o_row = o_head + (size_t)my_query * kHeadDim;
#pragma unroll
    for (int dblk = 0; dblk < 2; ++dblk)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f16x2 a = pack_rn(o_acc[dblk][4 * g + 0] * inv_l, o_acc[dblk][4 * g + 1] * inv_l);
            const f16x2 c = pack_rn(o_acc[dblk][4 * g + 2] * inv_l, o_acc[dblk][4 * g + 3] * inv_l);
            *reinterpret_cast<f16x4*>(o_row + 32 * dblk + 8 * g + 4 * half) =
                __builtin_shufflevector(a, c, 0, 1, 2, 3);
        }
}

template <bool kCausal, int kWaves>
hipError_t launch_forward(const void* q, const void* k, const void* v, void* o,
                          int64_t batch_heads, int64_t seq_len, float scale_log2,
                          hipStream_t stream) {
    const int64_t block_m = (int64_t)kWaves * kQueriesPerWave;
    const int64_t query_tiles = seq_len / block_m;
    const int64_t groups = batch_heads * query_tiles;
    hipLaunchKernelGGL((fa2_forward_d64_kernel<kCausal, kWaves>), dim3((unsigned)groups),
                       dim3(kWaves * 64), 0, stream,
                       static_cast<const _Float16*>(q), static_cast<const _Float16*>(k),
                       static_cast<const _Float16*>(v), static_cast<_Float16*>(o),
                       (int)seq_len, (int)query_tiles, scale_log2);
    return hipGetLastError();
}

// Queries per workgroup: 128 (4 waves) when the grid fills the chip, fewer waves per
// workgroup for small problems so that more CUs get work.
int choose_waves(int64_t batch_heads, int64_t seq_len) {
    constexpr int64_t kTargetGroups = 512;  // 2 per CU on 256 CUs
    if (batch_heads * (seq_len / 128) >= kTargetGroups) return 4;
    if (batch_heads * (seq_len / 64) >= kTargetGroups) return 2;
    return 1;
}

bool misaligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) != 0; }

}  // namespace

extern "C" int fa2_forward_production_128x128(const void* query, const void* key,
                                              const void* value, void* output, int64_t batch,
                                              int64_t heads, int64_t seq_len, int64_t head_dim,
                                              int causal, void* stream) {
    if (batch < 0 || heads < 0 || seq_len < 0 || head_dim < 0) return FA2_STATUS_NEGATIVE_DIMENSION;
    if (head_dim != kHeadDim) return FA2_STATUS_BAD_HEAD_DIM;
    if (seq_len % kQueryTileAlign != 0) return FA2_STATUS_BAD_SEQUENCE_LENGTH;
    if (batch == 0 || heads == 0 || seq_len == 0) return FA2_STATUS_SUCCESS;
    if (!query || !key || !value || !output) return FA2_STATUS_NULL_POINTER;
    if (misaligned(query) || misaligned(key) || misaligned(value) || misaligned(output))
        return FA2_STATUS_MISALIGNED;
    // Kernel indexing: seq_len and the query-tile count are int, the grid is 1-D.
    if (seq_len > (int64_t)INT32_MAX || batch > (int64_t)UINT32_MAX / heads)
        return FA2_STATUS_TOO_LARGE;
    const int64_t batch_heads = batch * heads;
    if (batch_heads > (int64_t)UINT32_MAX / (seq_len / kQueriesPerWave)) return FA2_STATUS_TOO_LARGE;

    const float scale = 1.0f / sqrtf((float)kHeadDim);           // reference :3040-3046
    const float scale_log2 = scale * 1.4426950408889634074f;     // fold log2(e) for exp2
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int waves = choose_waves(batch_heads, seq_len);
    hipError_t err;
    if (causal) {
        err = waves == 4   ? launch_forward<true, 4>(query, key, value, output, batch_heads, seq_len, scale_log2, s)
              : waves == 2 ? launch_forward<true, 2>(query, key, value, output, batch_heads, seq_len, scale_log2, s)
                           : launch_forward<true, 1>(query, key, value, output, batch_heads, seq_len, scale_log2, s);
    } else {
        err = waves == 4   ? launch_forward<false, 4>(query, key, value, output, batch_heads, seq_len, scale_log2, s)
              : waves == 2 ? launch_forward<false, 2>(query, key, value, output, batch_heads, seq_len, scale_log2, s)
                           : launch_forward<false, 1>(query, key, value, output, batch_heads, seq_len, scale_log2, s);
    }
    return err == hipSuccess ? FA2_STATUS_SUCCESS : FA2_STATUS_HIP_ERROR_BASE + (int)err;
}

extern "C" const char* fa2_status_string(int status) {
    switch (status) {
        case FA2_STATUS_SUCCESS: return "success";
        case FA2_STATUS_NULL_POINTER: return "null tensor pointer";
        case FA2_STATUS_NEGATIVE_DIMENSION: return "negative dimension";
        case FA2_STATUS_BAD_HEAD_DIM: return "head dimension must equal 64";
        case FA2_STATUS_BAD_SEQUENCE_LENGTH: return "sequence length must be divisible by 128";
        case FA2_STATUS_MISALIGNED: return "tensor pointer not 16-byte aligned";
        case FA2_STATUS_TOO_LARGE: return "problem too large for the kernel's launch grid";
        default: break;
    }
    if (status > FA2_STATUS_HIP_ERROR_BASE)
        return hipGetErrorString(static_cast<hipError_t>(status - FA2_STATUS_HIP_ERROR_BASE));
    return "unknown status";
}

extern "C" int fa2_abi_version(void) { return FA2_MI355X_ABI_VERSION; }
