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
//  * K/V tiles (64 keys x 64 dims, 8 KiB each) stream through four LDS stages by
//    direct-to-LDS buffer loads (no staging registers), fetched three tiles ahead
//    of use with one barrier per tile. A 16-byte-chunk XOR swizzle, applied on the
//    global side of the DMA, keeps the K reads (ds_read_b128) and the V transpose
//    reads free of bank conflicts.
//  * Software pipeline inside each wave: the scores of tile j+1 are computed
//    while the softmax of tile j runs, so MFMA and VALU work overlap.
//  * Causal mode stops the key loop at the diagonal, skips tiles a wave can never
//    see and masks only diagonal tiles (key > query -> -inf).
//  * Large problems run a wide variant with 64 queries per wave (two 32-query
//    blocks sharing each K and V^T fragment), which halves the LDS traffic per
//    FLOP: with random data the kernels run at the chip's power limit, and less
//    data movement buys clock.
//  * Workgroup ids are remapped so all query tiles of one (batch, head) land on the
//    same XCD (dispatch is round-robin over the 8 XCDs), keeping that head's K/V
//    resident in one L2; causal tiles run heaviest first, and the wide variant
//    runs a head's causal tiles T-1-p and p in one workgroup (T even), so every
//    workgroup streams the same number of key tiles.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#include <type_traits>
#include <atomic>

#include "fa2_mi355x.h"

namespace {

constexpr int kHeadDim = 64;
constexpr int kQueriesPerWave = 32;
constexpr int kKeysPerTile = 64;                          // BN
constexpr int kRowBytes = kHeadDim * 2;                   // 128 B per key row
constexpr int kTileBytes = kKeysPerTile * kRowBytes;      // 8 KiB
constexpr int kQueryTileAlign = 128;                      // reference kProductionBlockM/N
constexpr float kRescaleLog2 = 14.0f;                     // lazy-rescale threshold, log2 units
// A lane's probabilities are all <= 2^kRescaleLog2 when their sum is. The row sums
// add probability pairs in FP16 first, which stays finite for this bound:
// 2 * 2^14 = 2^15 < 65504.
constexpr float kTileSumBound = 16384.0f;                 // 2^kRescaleLog2
static_assert(kTileSumBound == 16384.0f && kRescaleLog2 == 14.0f, "kTileSumBound is 2^kRescaleLog2");
constexpr int64_t kMaxSeqLen = (int64_t)1 << 24;          // byte offsets in a head's slab fit in int32

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __fp16 fp16x4_lds __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define FA2_LDS __attribute__((address_space(3)))

// XOR applied to the 16-byte chunk index of key row `row` inside an LDS tile:
// chunk ^= b3 | (b0 ^ b2) << 1 | b1 << 2, with b_k bit k of the row. A tile row is
// 128 B; the mask keeps every LDS access of the kernel free of bank conflicts for
// 32 banks (128 B per pass) and for 64 banks (256 B per pass):
//  - K reads (ds_read_b128, A operand of K*Q^T): a pass covers MFMA rows 8g..8g+7
//    (or 16g..16g+15), i.e. key rows sigma(.) whose bits {0,1,3} (or {0,1,2,3})
//    take every value; the mask maps them to distinct (row parity, chunk) slots.
//  - V transpose reads (ds_read_b64_tr_b16): a 16-lane group reads rows 4a..4a+3
//    at one 32-byte column pair, two groups read the 4 pairs of one 64-byte quad;
//    bits 1-2 of the mask move the 4 rows to 4 pairs and b1 moves rows of equal
//    parity to opposite quads.
//  - Tile fills are LDS-DMA writes of 1 KiB contiguous per instruction.
__device__ __forceinline__ int tile_swizzle(int row) {
    return ((row >> 3) & 1) | (((row ^ (row >> 2)) & 1) << 1) | (((row >> 1) & 1) << 2);
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

// Buffer resource over one head's [seq_len, 64] FP16 slab (gfx9 descriptor word 3).
// Buffer loads take the slab base from SGPRs and a 32-bit per-lane offset, and
// return zeros outside num_records instead of faulting.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t head_resource(const void* base, int seq_len) {
    // num_records = seq_len * 128 reaches 2^31 at the largest seq_len: unsigned arithmetic.
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                            (int)((uint32_t)seq_len * (uint32_t)kRowBytes), 0x00020000);
}

// One LDS-DMA instruction (buffer_load_dwordx4 ... lds) moves 1 KiB: rows r0..r0+7
// of a K or V tile. Lane i writes LDS row r0 + i/8, chunk i%8 (the hardware writes
// lane i at M0 + 16*i), so it reads the global chunk the swizzle places there:
// logical chunk (i%8) ^ tile_swizzle(r0 + i/8). `lane_offset` is that lane's byte
// offset relative to row r0; it depends on r0 only through bit 3 of the row.
__device__ __forceinline__ int dma_lane_offset(int lane, int r0_bit3) {
    const int row = (lane >> 3) | (r0_bit3 << 3);
    return (lane >> 3) * kRowBytes + (((lane & 7) ^ tile_swizzle(row)) << 4);
}

__device__ __forceinline__ void dma_rows(__amdgpu_buffer_rsrc_t src, uint8_t* lds_rows,
                                         int lane_offset, int src_offset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(src, (FA2_LDS void*)lds_rows, 16, lane_offset,
                                             src_offset, 0, 0);
}

// Waits until at most `kPending` vector-memory instructions of this wave are in
// flight and its LDS reads are done, then joins the workgroup barrier. The caller
// passes the number of LDS-DMA instructions issued after the tile it needs.
template <int kPending>
__device__ __forceinline__ void wait_dma_and_barrier() {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kPending) : "memory");
}

// Causal head groups: with every XCD owning batch_heads / 8 whole heads, the XCD
// runs them a group at a time, and within a group the query tiles (or blocks) run
// heaviest first across all its heads: every head's last tile, then every head's
// second-to-last, and so on. A group has about as many tiles as an XCD has workgroup
// slots (32 CUs, two workgroups each), so its workgroups start on the same keys
// together and share its heads' K/V through L2, and the longest-first order drains
// the slots evenly: heads per group for T tiles per head is 64 / T, from 1 to 8.
// Head-major order (each head's tiles heaviest first, one head after another) instead
// starts the heavy tiles of an XCD's later heads only after light ones finish.
__device__ __forceinline__ uint32_t group_heads(uint32_t tiles_per_head) {
    return tiles_per_head >= 64 ? 1u : tiles_per_head >= 32 ? 2u : tiles_per_head >= 16 ? 4u : 8u;
}

// Workgroup -> (batch*head, work item) for grids of `tiles_per_head` items per head.
// Dispatch is round-robin over the 8 XCDs (id % 8), so every XCD gets a contiguous
// range of logical (head-major) items and the items of one head share that XCD's L2.
// `item` counts from the heaviest (item 0 = the last query tile of a head).
// Noncausal: the XCD's range in order. Causal: the range in level order (every head's
// item 0, then every head's item 1, ...), chunk by chunk when the range divides into
// chunks of group_heads(T) heads' worth of items (the head groups above when
// batch_heads is a multiple of 8), else as one chunk: a short last chunk would hold
// heavy items that start only after the earlier chunks have filled the slots. Where
// the XCD ranges split heads, a chunk's first and last head contribute only some
// levels; a binary search over the levels finds the slot's level from the count of
// the chunk's items below each level. Measured on MI355X (same process, bit-identical,
// fixed-size chunks -> this): -20% to -32% at B1 H66 N4096, B1 H72 N4096, B1 H80
// N4096, B1 H130 N2048, B1 H36 N4096, B1 H40 N4096. One chunk per XCD everywhere
// instead cost 1-3% where the chunks are whole (B16 H16 N4096, B1 H64 N4096): the
// XCD's L2 then holds more heads' K/V at once.
struct WorkItem {
    uint32_t bh, item;
};
template <bool kCausal>
__device__ __forceinline__ WorkItem xcd_work_item(uint32_t tiles_per_head) {
    const uint32_t T = tiles_per_head;
    const uint32_t groups = gridDim.x;
    const uint32_t xcd = blockIdx.x & 7u;
    const uint32_t slot = blockIdx.x >> 3;
    const uint32_t per_xcd = groups >> 3;
    const uint32_t extra = groups & 7u;
    const uint32_t xcd_begin = xcd * per_xcd + min(xcd, extra);
    if (!kCausal) {
        const uint32_t logical = xcd_begin + slot;
        const uint32_t bh = logical / T;
        return {bh, logical - bh * T};
    }
    const uint32_t count = per_xcd + (xcd < extra ? 1u : 0u);
    const uint32_t group_items = group_heads(T) * T;
    const uint32_t chunk_items = count % group_items == 0 ? group_items : count;
    const uint32_t chunk = slot / chunk_items;
    const uint32_t begin = xcd_begin + chunk * chunk_items;
    const uint32_t end = begin + chunk_items;  // exclusive
    const uint32_t rank = slot - chunk * chunk_items;  // position in level order
    const uint32_t head_first = begin / T, level_first = begin - head_first * T;  // its levels >= level_first
    const uint32_t head_last = (end - 1) / T, level_last = (end - 1) - head_last * T;  // its levels <= level_last
    // Items of the chunk on levels below k.
    auto below = [&](uint32_t k) -> uint32_t {
        if (head_first == head_last) return k <= level_first ? 0u : min(k, level_last + 1u) - level_first;
        const uint32_t full_heads = head_last - head_first - 1u;
        return full_heads * k + (k > level_first ? k - level_first : 0u) + min(k, level_last + 1u);
    };
    uint32_t lo = 0, hi = T;  // below(lo) <= rank < below(hi)
    while (hi - lo > 1u) {
        const uint32_t mid = (lo + hi) >> 1;
        if (below(mid) <= rank) lo = mid;
        else hi = mid;
    }
    const uint32_t r = rank - below(lo);  // among the heads that have level lo, in head order
    uint32_t bh;
    if (head_first == head_last) bh = head_first;
    else if (lo >= level_first) bh = head_first + r;  // the first head has this level
    else bh = head_first + 1u + r;
    return {bh, lo};
}

template <bool kCausal, int kWaves>
__global__ __launch_bounds__(kWaves * 64)
__attribute__((amdgpu_waves_per_eu(kWaves == 4 ? 2 : 1)))  // 4-wave groups: two waves per SIMD
void fa2_forward_d64_kernel(const _Float16* __restrict__ query,
                            const _Float16* __restrict__ key,
                            const _Float16* __restrict__ value,
                            _Float16* __restrict__ output,
                            int seq_len, int num_query_tiles, float scale_log2) {
    constexpr int kBlockM = kWaves * kQueriesPerWave;
    // Tile t (K then V, 16 KiB) lives in stage t % 4. Iteration j reads V of tile j
    // and K of tile j+1, tile j+2 is landing and tile j+3 is being fetched, so the
    // fetch runs two iterations ahead of its use with one barrier per tile. Four
    // separate arrays let the compiler see that a fetch and a read of another stage
    // are independent.
    constexpr int kStageBytes = 2 * kTileBytes;
    constexpr int kDmaPerTile = 2 * kTileBytes / 1024 / kWaves;  // LDS-DMA instructions per wave
    __shared__ __attribute__((aligned(1024))) uint8_t stage0[kStageBytes];
    __shared__ __attribute__((aligned(1024))) uint8_t stage1[kStageBytes];
    __shared__ __attribute__((aligned(1024))) uint8_t stage2[kStageBytes];
    __shared__ __attribute__((aligned(1024))) uint8_t stage3[kStageBytes];
    auto stage_at = [&](int st) -> uint8_t* {
        return st == 0 ? stage0 : st == 1 ? stage1 : st == 2 ? stage2 : stage3;
    };

    const int tid = threadIdx.x;
    // Wave index in an SGPR: it selects buffer descriptors and LDS-DMA bases.
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int lq = lane & 31;   // query column owned by this lane
    const int half = lane >> 5; // which 16 of each 32 keys this lane holds

    // Workgroup -> (batch*head, query tile): XCD-contiguous, causal tiles heaviest
    // first in head groups. Measured on MI355X against head-major order (same process,
    // bit-identical): -17% at B1 H32 N4096, -23% at B4 H16 N2048 and B8 H16 N1024, -15%
    // at B16 H16 N512, -11% at B1 H16 N4096; unchanged with one head per XCD.
    const WorkItem work = xcd_work_item<kCausal>((uint32_t)num_query_tiles);
    const uint32_t bh = work.bh;
    const uint32_t qtile = kCausal ? (uint32_t)num_query_tiles - 1u - work.item : work.item;

    const size_t head_offset = (size_t)bh * (size_t)seq_len * kHeadDim;
    const _Float16* __restrict__ q_head = query + head_offset;
    const __amdgpu_buffer_rsrc_t k_head = head_resource(key + head_offset, seq_len);
    const __amdgpu_buffer_rsrc_t v_head = head_resource(value + head_offset, seq_len);
    _Float16* __restrict__ o_head = output + head_offset;

    const int q_block = (int)qtile * kBlockM;
    const int q_wave = q_block + wave * kQueriesPerWave;
    const int my_query = q_wave + lq;

    // Key tiles the workgroup streams, and the last one this wave can see.
    const int num_tiles = kCausal ? (q_block + kBlockM - 1) / kKeysPerTile + 1
                                  : seq_len / kKeysPerTile;
    const int wave_last_tile = kCausal ? (q_wave + kQueriesPerWave - 1) / kKeysPerTile
                                       : num_tiles - 1;

    // LDS-DMA of tile t into a stage: this wave issues instructions n = wave + x*kWaves
    // of the 16 (8 per matrix, 8 rows each).
    const int dma_off[2] = {dma_lane_offset(lane, 0), dma_lane_offset(lane, 1)};
    auto dma_tile = [&](int t, uint8_t* stage) {
#pragma unroll
        for (int x = 0; x < kDmaPerTile; ++x) {
            const int n = wave + x * kWaves;
            const int m = n >> 3;
            const int r0 = (n & 7) * 8;
            dma_rows(m ? v_head : k_head, stage + m * kTileBytes + r0 * kRowBytes, dma_off[n & 1],
                     t * kTileBytes + r0 * kRowBytes);
        }
    };
    // Tiles 0..2 start landing while Q is loaded.
    dma_tile(0, stage0);
    if (num_tiles > 1) dma_tile(1, stage1);
    if (num_tiles > 2) dma_tile(2, stage2);

    // Q^T as the B operand of K*Q^T: lane holds dims 16ks + 8*half + 0..7 of its query.
    f16x8 q_frag[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
        q_frag[ks] = *reinterpret_cast<const f16x8*>(q_head + (size_t)my_query * kHeadDim +
                                                      ks * 16 + half * 8);

    // Per-lane LDS byte offsets.
    // K (A operand): MFMA row lq reads key row sigma(lq) (+32 rows for block 1) at
    // chunk 2ks + half.
    const int k_row = key_of_mfma_row(lq);
    const int k_swz = tile_swizzle(k_row);
    int k_off[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) k_off[ks] = k_row * kRowBytes + (((2 * ks + half) ^ k_swz) << 4);
    // V^T (A operand) through transpose reads. In a 16-lane group g, lane i reads 4
    // halves at key row base + i/4, dims d0 + 4*(i%4); the read returns, to lane i,
    // dim d0 + i at keys base..base+3. Row base = 32b + 16t + 8*half + 4r; the
    // swizzle of that row depends on the lane and on r only.
    const int grp = lane >> 4;
    const int i16 = lane & 15;
    int v_off[2][2];  // [r][dblk]
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int dblk = 0; dblk < 2; ++dblk) {
            const int row = 8 * half + 4 * r + (i16 >> 2);
            const int chunk = 4 * dblk + 2 * (grp & 1) + ((i16 & 3) >> 1);
            v_off[r][dblk] = row * kRowBytes + ((chunk ^ tile_swizzle(row)) << 4) + 8 * (i16 & 1);
        }

    f32x16 o_acc[2];
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
        for (int i = 0; i < 16; ++i) o_acc[d][i] = 0.0f;
    float m_run = -INFINITY;  // running max of raw scores (unscaled) for my_query
    float l_run = 0.0f;       // this lane's share of the running softmax denominator
    const f16x2 ones = {(_Float16)1.0f, (_Float16)1.0f};

    // K fragments of a tile: block b (keys 32b..32b+31), k-step ks (dims 16ks..16ks+15).
    auto load_k = [&](const uint8_t* k_lds, f16x8 (&kf)[2][4]) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int b = 0; b < 2; ++b)
                kf[b][ks] = *reinterpret_cast<const f16x8*>(k_lds + b * 32 * kRowBytes + k_off[ks]);
    };
    // V^T fragment of P.V MFMA k of a tile: block k/4, 16-key half (k/2)%2, d-block k%2.
    auto load_v = [&](const uint8_t* v_lds, int k) -> f16x8 {
        const int row_base = (32 * (k >> 2) + 16 * ((k >> 1) & 1)) * kRowBytes;
        const f16x4 v_lo = lds_read_transposed(v_lds + row_base + v_off[0][k & 1]);
        const f16x4 v_hi = lds_read_transposed(v_lds + row_base + v_off[1][k & 1]);
        return __builtin_shufflevector(v_lo, v_hi, 0, 1, 2, 3, 4, 5, 6, 7);
    };
    // S^T MFMA k of a tile: block k%2, k-step k/2 (the block's chain starts at k < 2).
    auto score_mfma = [&](const f16x8 (&kf)[2][4], int k, f32x16 (&s)[2]) {
        const f32x16 zero = {};
        const int b = k & 1, ks = k >> 1;
        s[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[b][ks], q_frag[ks], ks == 0 ? zero : s[b], 0, 0, 0);
    };

    // Causal mask of tile t: register i of block b holds key 64t + 32b + 16(i/8) +
    // 8*half + i%8; keys after my_query become -inf. Only tiles that reach past the
    // wave's first query need it.
    auto mask = [&](int t, f32x16 (&s)[2]) {
        if (!kCausal || t * kKeysPerTile + kKeysPerTile - 1 <= q_wave) return;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int key_index = t * kKeysPerTile + 32 * b + 16 * (i >> 3) + 8 * half + (i & 7);
                if (key_index > my_query) s[b][i] = -INFINITY;
            }
    };

    // Lazy rescale: the running max moves only when some query's tile max exceeds
    // it by more than kRescaleLog2 (log2 units), so probabilities stay below
    // 2^kRescaleLog2 and O, l share one (possibly stale) max - O / l is unchanged.
    // The first tile always moves it (m_run = -inf gives alpha = 0). l is rescaled
    // here; O by the caller (rarely needed: behind a wave-uniform branch placed where
    // O is not being accumulated). Returns whether O needs it and sets `alpha`.
    auto decide_rescale = [&](float tile_max, float& alpha) -> bool {
        tile_max = max_across_halves(tile_max);
        const bool grow = tile_max * scale_log2 > m_run * scale_log2 + kRescaleLog2;
        const bool any_grow = __builtin_amdgcn_ballot_w64(grow) != 0;
        const float m_new = any_grow ? fmaxf(m_run, tile_max) : m_run;
        alpha = m_new == m_run ? 1.0f : __builtin_amdgcn_exp2f((m_run - m_new) * scale_log2);
        l_run *= alpha;
        m_run = m_new;
        return any_grow;
    };
    auto partial_max = [&](const f32x16& sb, int i0, int n, float m) {
#pragma unroll
        for (int i = 0; i < n; i += 2) m = fmaxf(fmaxf(m, sb[i0 + i]), sb[i0 + i + 1]);
        return m;
    };
    auto rescale_o = [&](float alpha) {
#pragma unroll
        for (int d = 0; d < 2; ++d)
#pragma unroll
            for (int i = 0; i < 16; ++i) o_acc[d][i] *= alpha;
    };

    // One exp pair: p = 2^(s*scale*log2e - m*scale*log2e) for accumulator registers
    // 2q, 2q+1 of a block, rounded to FP16 (nearest). Every second pair adds the
    // last two pairs to the row sum: one packed FP16 add, then v_dot2_f32_f16
    // against 1.0 into the FP32 sum (v_dot2 does not overlap MFMA execution,
    // v_pk_add_f16 does, so this halves the dot2s at one extra FP16 rounding).
    auto exp_pair = [&](const f32x16& sb, int q, float m_scaled, f16x2 (&pk)[8], float& sum) {
        pk[q] = pack_rn(__builtin_amdgcn_exp2f(fmaf(sb[2 * q], scale_log2, -m_scaled)),
                        __builtin_amdgcn_exp2f(fmaf(sb[2 * q + 1], scale_log2, -m_scaled)));
        if (q & 1) sum = __builtin_amdgcn_fdot2(pk[q - 1] + pk[q], ones, sum, false);
    };
    // The 8 pairs of a block as the B operands of its two P.V MFMAs (16 keys each).
    auto assemble = [&](const f16x2 (&pk)[8], f16x8 (&p)[2]) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const f16x4 lo = __builtin_shufflevector(pk[4 * t], pk[4 * t + 1], 0, 1, 2, 3);
            const f16x4 hi = __builtin_shufflevector(pk[4 * t + 2], pk[4 * t + 3], 0, 1, 2, 3);
            p[t] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        }
    };
    // Probabilities are computed against the running max before the tile's own max
    // is known (the "stale" max). A lane's probabilities are all <= 2^kRescaleLog2
    // when their sum is, so one compare of the tile's row sum replaces the row max
    // in the common case; only when some lane's sum exceeds the bound is the exact
    // tile max taken (decide_rescale) and the tile's probabilities recomputed.
    // Redo tile `s` after a failed check: exact max, rescale of l and O, and both
    // blocks' probabilities against the new max. Returns the tile's lane sum.
    auto refresh_tile = [&](const f32x16 (&s)[2], f16x8 (&p0)[2], f16x8 (&p1)[2], float tile_sum) -> float {
        float alpha;
        const float tile_max = partial_max(s[1], 0, 16, partial_max(s[0], 0, 16, -INFINITY));
        if (!decide_rescale(tile_max, alpha)) return tile_sum;  // every probability is <= 2^kRescaleLog2
        rescale_o(alpha);
        const float m_scaled = m_run * scale_log2;
        float sum = 0.0f;
        f16x2 pk[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) exp_pair(s[0], q, m_scaled, pk, sum);
        assemble(pk, p0);
#pragma unroll
        for (int q = 0; q < 8; ++q) exp_pair(s[1], q, m_scaled, pk, sum);
        assemble(pk, p1);
        return sum;
    };

    // Prologue: tiles 0..2 landed; scores, exact max and block-0 P of tile 0.
    __syncthreads();  // waits for every outstanding DMA (tiles 0..2) and Q
    f32x16 s_a[2], s_b[2];
    f16x8 p_lo[2];        // FP16 P of block 0 of the tile being finished
    float sum_lo = 0.0f;  // its lane sum, not yet in l_run
    {
        f16x8 kf[2][4];
        load_k(stage0, kf);
#pragma unroll
        for (int k = 0; k < 8; ++k) score_mfma(kf, k, s_a);
        mask(0, s_a);
        float alpha;
        const float tile_max = partial_max(s_a[1], 0, 16, partial_max(s_a[0], 0, 16, -INFINITY));
        if (decide_rescale(tile_max, alpha)) rescale_o(alpha);
        f16x2 pk[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) exp_pair(s_a[0], q, m_run * scale_log2, pk, sum_lo);
        assemble(pk, p_lo);
    }

    // Iteration j finishes tile j (cur) and starts tile j+1 (next) in two phases of
    // eight MFMAs, each slot with one exp pair beside its MFMA:
    //   phase 1: S^T of tile j+1 (8 MFMAs)  | exp of block 1 of tile j, V^T reads of tile j
    //   check of tile j (rarely: exact max and recompute)
    //   phase 2: P.V of tile j (8 MFMAs)    | exp of block 0 of tile j+1
    //
    // Steady state: tiles j and j+1 are unmasked and seen by every wave and tile j+3
    // exists. Stages are compile-time (j % 4 == kStage); the order of MFMA, VALU and
    // LDS reads is fixed by scheduling fences, one MFMA per slot.
    auto steady = [&](int j, auto stage_tag, f32x16 (&cur)[2], f32x16 (&next)[2]) {
        constexpr int kStage = decltype(stage_tag)::value;
        uint8_t* const st_cur = kStage == 0 ? stage0 : kStage == 1 ? stage1 : kStage == 2 ? stage2 : stage3;
        uint8_t* const st_next = kStage == 3 ? stage0 : kStage == 0 ? stage1 : kStage == 1 ? stage2 : stage3;
        uint8_t* const st_fetch = kStage == 1 ? stage0 : kStage == 2 ? stage1 : kStage == 3 ? stage2 : stage3;
        dma_tile(j + 3, st_fetch);
        f16x8 kf[2][4];
        load_k(st_next, kf);
        const uint8_t* v_lds = st_cur + kTileBytes;
        __builtin_amdgcn_sched_barrier(0);

        // Phase 1: slot k = score MFMA k of tile j+1 (block 0's chain first, so it is
        // complete before phase 2 reads it) + exp pair k of block 1 of tile j + the
        // transpose reads of P.V MFMA k of tile j.
        // Phase 1 runs at raised wave priority: its MFMAs are independent of
        // the other wave's softmax, so the arbiter should favour them.
        __builtin_amdgcn_s_setprio(1);
        const float m_cur = m_run * scale_log2;
        f16x2 pk_hi[8];
        float sum_hi = 0.0f;
        f16x8 vf[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            score_mfma(kf, ((k & 3) << 1) | (k >> 2), next);
            exp_pair(cur[1], k, m_cur, pk_hi, sum_hi);
            vf[k] = load_v(v_lds, k);
            __builtin_amdgcn_sched_barrier(0);
        }
        f16x8 p_hi[2];
        assemble(pk_hi, p_hi);
        float tile_sum = sum_lo + sum_hi;
        if (__builtin_amdgcn_ballot_w64(tile_sum > kTileSumBound) != 0)
            tile_sum = refresh_tile(cur, p_lo, p_hi, tile_sum);
        l_run += tile_sum;
        __builtin_amdgcn_sched_barrier(0);

        __builtin_amdgcn_s_setprio(0);
        // Phase 2: P.V MFMAs of tile j (block 0 with p_lo, block 1 with p_hi) beside
        // the exp of block 0 of tile j+1 against the current max.
        const float m_next = m_run * scale_log2;
        f16x2 pk_lo[8];
        sum_lo = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const f16x8& pf = (k < 4) ? p_lo[(k >> 1) & 1] : p_hi[(k >> 1) & 1];
            o_acc[k & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[k], pf, o_acc[k & 1], 0, 0, 0);
            exp_pair(next[0], k, m_next, pk_lo, sum_lo);
            __builtin_amdgcn_sched_barrier(0);
        }
        assemble(pk_lo, p_lo);
        // Tile j+2 must have landed (only tile j+3's DMAs may be in flight).
        wait_dma_and_barrier<kDmaPerTile>();
    };

    // Any iteration: the last tiles, causal diagonal tiles, tiles a wave of a causal
    // workgroup does not see, and steady iterations that do not start a group of 4.
    auto generic = [&](int j, f32x16 (&cur)[2], f32x16 (&next)[2]) {
        const bool active = j <= wave_last_tile;
        const bool next_active = j + 1 < num_tiles && j + 1 <= wave_last_tile;
        if (j + 3 < num_tiles) dma_tile(j + 3, stage_at((j + 3) & 3));
        const uint8_t* v_lds = stage_at(j & 3) + kTileBytes;
        if (active) {
            f16x2 pk[8];
            float sum_hi = 0.0f;
#pragma unroll
            for (int q = 0; q < 8; ++q) exp_pair(cur[1], q, m_run * scale_log2, pk, sum_hi);
            f16x8 p_hi[2];
            assemble(pk, p_hi);
            float tile_sum = sum_lo + sum_hi;
            if (__builtin_amdgcn_ballot_w64(tile_sum > kTileSumBound) != 0)
                tile_sum = refresh_tile(cur, p_lo, p_hi, tile_sum);
            l_run += tile_sum;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const f16x8& pf = (k < 4) ? p_lo[(k >> 1) & 1] : p_hi[(k >> 1) & 1];
                o_acc[k & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(load_v(v_lds, k), pf, o_acc[k & 1], 0, 0, 0);
            }
        }
        if (next_active) {
            f16x8 kf[2][4];
            load_k(stage_at((j + 1) & 3), kf);
#pragma unroll
            for (int k = 0; k < 8; ++k) score_mfma(kf, k, next);
            mask(j + 1, next);
            f16x2 pk[8];
            sum_lo = 0.0f;
#pragma unroll
            for (int q = 0; q < 8; ++q) exp_pair(next[0], q, m_run * scale_log2, pk, sum_lo);
            assemble(pk, p_lo);
        }
        __syncthreads();  // waits for every outstanding DMA
    };

    // Steady iterations need tiles j and j+1 unmasked for wave 0 (the workgroup's
    // first query); they run from j = 0 in groups of four plus a remainder of up to
    // three, so that j % 4 (the stage) is known at compile time. The last tile and
    // the causal diagonal tiles take the generic iteration.
    const int first_masked_tile = kCausal ? q_block / kKeysPerTile : num_tiles;
    const int steady_end = max(0, min(first_masked_tile - 1, num_tiles - 3));
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    using S3 = std::integral_constant<int, 3>;
    int j = 0;
    for (; j + 4 <= steady_end; j += 4) {
        steady(j, S0{}, s_a, s_b);
        steady(j + 1, S1{}, s_b, s_a);
        steady(j + 2, S2{}, s_a, s_b);
        steady(j + 3, S3{}, s_b, s_a);
    }
    const int rest = steady_end - j;  // 0..3
    if (rest >= 1) steady(j, S0{}, s_a, s_b);
    if (rest >= 2) steady(j + 1, S1{}, s_b, s_a);
    if (rest >= 3) steady(j + 2, S2{}, s_a, s_b);
    j += rest;
    bool flipped = (rest & 1) != 0;
    for (; j < num_tiles; ++j) {
        if (flipped) generic(j, s_b, s_a);
        else generic(j, s_a, s_b);
        flipped = !flipped;
    }

    // Epilogue: O = O^T / l. Accumulator i of d-block dblk holds dim
    // 32*dblk + 8*(i/4) + 4*half + i%4 of my_query, i.e. 16-byte chunk 4*dblk + i/4 of
    // its row. The wave's 32 rows go through its 4 KiB of stage 3 (free after the last
    // tile's barrier; chunk c of row r at c ^ (r & 7)) and are stored as whole rows.
    const float inv_l = 1.0f / sum_across_halves(l_run);
    static_assert(kWaves * kQueriesPerWave * kRowBytes <= kStageBytes, "every wave's output block fits stage 3");
    uint8_t* const out_lds = stage3 + wave * (kQueriesPerWave * kRowBytes);
#pragma unroll
    for (int dblk = 0; dblk < 2; ++dblk)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f16x2 a = pack_rn(o_acc[dblk][4 * g + 0] * inv_l, o_acc[dblk][4 * g + 1] * inv_l);
            const f16x2 c = pack_rn(o_acc[dblk][4 * g + 2] * inv_l, o_acc[dblk][4 * g + 3] * inv_l);
            const int chunk = 4 * dblk + g;
            *reinterpret_cast<f16x4*>(out_lds + lq * kRowBytes + ((chunk ^ (lq & 7)) << 4) + 8 * half) =
                __builtin_shufflevector(a, c, 0, 1, 2, 3);
        }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = 8 * r + (lane >> 3);
        const int chunk = lane & 7;
        const f16x8 v = *reinterpret_cast<const f16x8*>(out_lds + row * kRowBytes + ((chunk ^ (row & 7)) << 4));
        *reinterpret_cast<f16x8*>(o_head + (size_t)(q_wave + row) * kHeadDim + 8 * chunk) = v;
    }
}

// LDS-DMA through inline assembly: M0 = LDS destination of lane 0 (wave-uniform),
// then buffer_load_dwordx4 ... lds. The compiler does not track these loads, so it
// adds no waits for them; the kernel waits with explicit vmcnt. M0 is a reserved
// register that the compiler sets before each of its own uses, so listing it as
// clobbered is only documentation (clang warns about reserved clobbers).
//  - dma16_asm: tile offset in the scalar offset, for tiles inside the slab.
//  - dma16_asm_checked: the whole byte offset in the VGPR offset, which the buffer
//    unit checks against num_records (the scalar offset is not checked), so rows at
//    or past seq_len read as zeros: used for a partial last key tile.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16_asm(u32x4 src, uint32_t lds_addr, int lane_offset,
                                          int src_offset) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :: "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(lane_offset), "s"(src),
                    "s"(__builtin_amdgcn_readfirstlane(src_offset))
                 : "memory", "m0");
}
__device__ __forceinline__ void dma16_asm_checked(u32x4 src, uint32_t lds_addr, int offset) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :: "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(offset), "s"(src)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// Buffer descriptor (base, stride 0, num_records, gfx9 word 3) in SGPRs, as an
// inline-assembly operand.
__device__ __forceinline__ u32x4 head_descriptor(const void* base, int seq_len) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    u32x4 d;
    d[0] = __builtin_amdgcn_readfirstlane((uint32_t)a);
    d[1] = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xffffu);
    d[2] = (uint32_t)seq_len * (uint32_t)kRowBytes;  // up to 2^31: unsigned arithmetic
    d[3] = 0x00020000u;
    return d;
}

__device__ __forceinline__ uint32_t lds_address(const void* p) {
    return (uint32_t)(uintptr_t)(FA2_LDS const void*)p;
}

// Key-split variant for problems too small to fill the chip with 128-query
// workgroups, and for sequence lengths that are not a multiple of 128 (any multiple
// of 16: the last query block and the last key tile may be partial). A workgroup
// owns one 32-query block; its kSplit waves each stream a contiguous share of the
// key tiles (kBlocks 32-key blocks each) that block sees, through two LDS stages
// of their own (each wave fetches and reads only its own stages, so the key loop
// has no workgroup barrier), and keep their own running max, sum and O. At the end
// the partial results are merged through LDS:
//   m = max_w m_w,  l = sum_w l_w 2^((m_w - m) s log2e),  O = sum_w O_w 2^(...) / l,
// and the FP16 output tile is staged in LDS so that the stores write whole 128-byte rows
// (measured 0-2% faster than 8-byte stores scattered over the 32 rows).
template <bool kCausal, bool kPartial, int kSplit, int kBlocks>
__global__ __launch_bounds__(kSplit * 64) void fa2_forward_splitk_kernel(const _Float16* __restrict__ query,
                                                                 const _Float16* __restrict__ key,
                                                                 const _Float16* __restrict__ value,
                                                                 _Float16* __restrict__ output,
                                                                 int seq_len, int num_query_blocks,
                                                                 float scale_log2) {
    constexpr int kTileKeys = 32 * kBlocks;
    constexpr int kTileBytesW = kTileKeys * kRowBytes;
    constexpr int kStageBytes = 2 * kTileBytesW;            // K tile then V tile
    constexpr int kDmaPerMatrix = kTileBytesW / 1024;        // 1 KiB = 8 rows per instruction
    constexpr int kDmaPerTile = 2 * kDmaPerMatrix;           // one wave fetches whole tiles
    constexpr int kMergeBytes = kSplit * (8 * 64 * 16 + 2 * 64 * 4);
    constexpr int kQBytes = kQueriesPerWave * kRowBytes;  // the block's Q rows, 4 KiB per wave
    constexpr int kWaveBytes = 2 * kStageBytes + kQBytes;
    constexpr int kSmemBytes = kSplit * kWaveBytes > kMergeBytes ? kSplit * kWaveBytes : kMergeBytes;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kSmemBytes];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int lq = lane & 31;
    const int half = lane >> 5;

    // Workgroup -> (batch*head, query block): XCD-contiguous, head by head, causal
    // blocks heaviest first. (The 128-query kernel's level order measured 0 to +4% at
    // B1 H24 N1024, B1 H32 N1024, B4 H8 N1024, B1 H16 N2048, B1 H12 N2048 and -4% at
    // B1 H36 N1024: these grids are a few rounds of short workgroups whose keys are
    // already split over four waves.)
    const WorkItem work = xcd_work_item<false>((uint32_t)num_query_blocks);
    const uint32_t bh = work.bh;
    const uint32_t qblock = kCausal ? (uint32_t)num_query_blocks - 1u - work.item : work.item;

    const size_t head_offset = (size_t)bh * (size_t)seq_len * kHeadDim;
    const _Float16* __restrict__ q_head = query + head_offset;
    const u32x4 k_head = head_descriptor(key + head_offset, seq_len);
    const u32x4 v_head = head_descriptor(value + head_offset, seq_len);
    _Float16* __restrict__ o_head = output + head_offset;

    const int q0 = (int)qblock * kQueriesPerWave;
    const int my_query = q0 + lq;
    const bool query_valid = !kPartial || my_query < seq_len;
    const int visible_tiles = kCausal ? (q0 + kQueriesPerWave - 1) / kTileKeys + 1
                                      : (seq_len + kTileKeys - 1) / kTileKeys;
    const int t_begin = wave * visible_tiles / kSplit;
    const int t_end = (wave + 1) * visible_tiles / kSplit;

    uint8_t* const my_stages = smem + wave * kWaveBytes;
    const uint32_t my_stages_addr = lds_address(my_stages);
    const int dma_off[2] = {dma_lane_offset(lane, 0), dma_lane_offset(lane, 1)};
    auto dma_tile = [&](int t, int st) {
        const bool partial = kPartial && (t + 1) * kTileKeys > seq_len;  // wave-uniform
#pragma unroll
        for (int n = 0; n < kDmaPerTile; ++n) {
            const int m = n / kDmaPerMatrix;
            const int r0 = (n % kDmaPerMatrix) * 8;
            const uint32_t lds = my_stages_addr + (uint32_t)(st * kStageBytes + m * kTileBytesW + r0 * kRowBytes);
            const int src = t * kTileBytesW + r0 * kRowBytes;
            const int off = dma_off[(r0 >> 3) & 1];
            if (partial) dma16_asm_checked(m ? v_head : k_head, lds, off + src);
            else dma16_asm(m ? v_head : k_head, lds, off, src);
        }
    };

    // Q rows of the block go to this wave's LDS area by LDS-DMA ahead of the first key
    // tile, so the first tile's wait covers them; the fragments are read from LDS after
    // it. (Loads into registers would make the compiler wait for them with a vmcnt that
    // also counts the key-tile DMAs issued after them.) Rows past seq_len read as zeros,
    // so lanes past the last query (partial block) score a zero query.
    const u32x4 q_desc = head_descriptor(q_head, seq_len);
    uint8_t* const my_q = my_stages + 2 * kStageBytes;
    const uint32_t my_q_addr = my_stages_addr + 2 * kStageBytes;
#pragma unroll
    for (int n = 0; n < kQBytes / 1024; ++n) {
        const int r0 = n * 8;
        const int src = (q0 + r0) * kRowBytes;
        if (kPartial) dma16_asm_checked(q_desc, my_q_addr + (uint32_t)(r0 * kRowBytes), dma_off[n & 1] + src);
        else dma16_asm(q_desc, my_q_addr + (uint32_t)(r0 * kRowBytes), dma_off[n & 1], src);
    }
    if (t_begin < t_end) dma_tile(t_begin, 0);
    const int q_swz = tile_swizzle(lq);
    f16x8 q_frag[4];

    const int k_row = key_of_mfma_row(lq);
    const int k_swz = tile_swizzle(k_row);
    int k_off[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) k_off[ks] = k_row * kRowBytes + (((2 * ks + half) ^ k_swz) << 4);
    const int grp = lane >> 4;
    const int i16 = lane & 15;
    int v_off[2][2];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int dblk = 0; dblk < 2; ++dblk) {
            const int row = 8 * half + 4 * r + (i16 >> 2);
            const int chunk = 4 * dblk + 2 * (grp & 1) + ((i16 & 3) >> 1);
            v_off[r][dblk] = row * kRowBytes + ((chunk ^ tile_swizzle(row)) << 4) + 8 * (i16 & 1);
        }

    f32x16 o_acc[2];
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
        for (int i = 0; i < 16; ++i) o_acc[d][i] = 0.0f;
    float m_run = -INFINITY;
    float l_run = 0.0f;
    const f16x2 ones = {(_Float16)1.0f, (_Float16)1.0f};

    // Exact tile max and lazy rescale of l and O; returns whether the max moved.
    auto exact_max_update = [&](const f32x16 (&s)[kBlocks]) -> bool {
        float tile_max = -INFINITY;
#pragma unroll
        for (int b = 0; b < kBlocks; ++b)
#pragma unroll
            for (int i = 0; i < 16; i += 2) tile_max = fmaxf(fmaxf(tile_max, s[b][i]), s[b][i + 1]);
        tile_max = max_across_halves(tile_max);
        const bool grow = tile_max * scale_log2 > m_run * scale_log2 + kRescaleLog2;
        if (__builtin_amdgcn_ballot_w64(grow) == 0) return false;
        const float m_new = fmaxf(m_run, tile_max);
        const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * scale_log2);
        l_run *= alpha;
#pragma unroll
        for (int d = 0; d < 2; ++d)
#pragma unroll
            for (int i = 0; i < 16; ++i) o_acc[d][i] *= alpha;
        m_run = m_new;
        return true;
    };
    // FP16 probabilities of a tile against the running max as P.V B operands; returns
    // the lane sum (pairs added in FP16, then v_dot2 against 1.0 into FP32).
    auto tile_probs = [&](const f32x16 (&s)[kBlocks], f16x8 (&pf)[kBlocks][2]) -> float {
        const float m_scaled = m_run * scale_log2;
        float sum = 0.0f;
#pragma unroll
        for (int b = 0; b < kBlocks; ++b) {
            f16x2 pk[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                pk[q] = pack_rn(__builtin_amdgcn_exp2f(fmaf(s[b][2 * q], scale_log2, -m_scaled)),
                                __builtin_amdgcn_exp2f(fmaf(s[b][2 * q + 1], scale_log2, -m_scaled)));
                if (q & 1) sum = __builtin_amdgcn_fdot2(pk[q - 1] + pk[q], ones, sum, false);
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const f16x4 lo = __builtin_shufflevector(pk[4 * h], pk[4 * h + 1], 0, 1, 2, 3);
                const f16x4 hi = __builtin_shufflevector(pk[4 * h + 2], pk[4 * h + 3], 0, 1, 2, 3);
                pf[b][h] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
            }
        }
        return sum;
    };

    for (int t = t_begin; t < t_end; ++t) {
        const int st = (t - t_begin) & 1;
        if (t + 1 < t_end) {
            dma_tile(t + 1, st ^ 1);
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kDmaPerTile) : "memory");  // tile t landed
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        const uint8_t* k_lds = my_stages + st * kStageBytes;
        const uint8_t* v_lds = k_lds + kTileBytesW;
        if (t == t_begin) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                q_frag[ks] = *reinterpret_cast<const f16x8*>(my_q + lq * kRowBytes + (((2 * ks + half) ^ q_swz) << 4));
        }

        // S^T = K Q^T for the tile's 32-key blocks.
        f16x8 kf[kBlocks][4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int b = 0; b < kBlocks; ++b)
                kf[b][ks] = *reinterpret_cast<const f16x8*>(k_lds + b * 32 * kRowBytes + k_off[ks]);
        f32x16 sc[kBlocks];
        const f32x16 zero = {};
#pragma unroll
        for (int b = 0; b < kBlocks; ++b) sc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[b][0], q_frag[0], zero, 0, 0, 0);
#pragma unroll
        for (int ks = 1; ks < 4; ++ks)
#pragma unroll
            for (int b = 0; b < kBlocks; ++b)
                sc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[b][ks], q_frag[ks], sc[b], 0, 0, 0);

        // Causal mask on tiles reaching past the block's first query; keys at or
        // past seq_len (zeros from the DMA) on a partial last tile.
        const bool causal_tile = kCausal && t * kTileKeys + kTileKeys - 1 > q0;
        if (causal_tile || (kPartial && (t + 1) * kTileKeys > seq_len)) {
#pragma unroll
            for (int b = 0; b < kBlocks; ++b)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int key_index = t * kTileKeys + 32 * b + 16 * (i >> 3) + 8 * half + (i & 7);
                    if ((kCausal && key_index > my_query) || (kPartial && key_index >= seq_len))
                        sc[b][i] = -INFINITY;
                }
        }

        // Online softmax with the lazy rescale (bound 2^kRescaleLog2). The first tile
        // of the wave takes the exact max; later tiles use the running max and check
        // the lane sums (every probability is <= 2^kRescaleLog2 when its lane's sum is), taking
        // the exact max and recomputing only when a sum exceeds the bound.
        f16x8 pf[kBlocks][2];
        const bool first = t == t_begin;
        if (first) exact_max_update(sc);
        float tile_sum = tile_probs(sc, pf);
        if (!first && __builtin_amdgcn_ballot_w64(tile_sum > kTileSumBound) != 0) {
            if (exact_max_update(sc)) tile_sum = tile_probs(sc, pf);
        }
        l_run += tile_sum;

        // O^T += V^T P^T.
#pragma unroll
        for (int k = 0; k < 4 * kBlocks; ++k) {
            const int row_base = (32 * (k >> 2) + 16 * ((k >> 1) & 1)) * kRowBytes;
            const f16x4 v_lo = lds_read_transposed(v_lds + row_base + v_off[0][k & 1]);
            const f16x4 v_hi = lds_read_transposed(v_lds + row_base + v_off[1][k & 1]);
            const f16x8 vf = __builtin_shufflevector(v_lo, v_hi, 0, 1, 2, 3, 4, 5, 6, 7);
            o_acc[k & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[k >> 2][(k >> 1) & 1], o_acc[k & 1], 0, 0, 0);
        }
    }

    // Merge the partial results (stages are free once every wave is done). A wave without
    // key tiles still has its Q DMA to wait for before the merge reuses that LDS.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    float* red_o = reinterpret_cast<float*>(smem);                  // [wave][8][64 lanes][4]
    float* red_m = red_o + kSplit * 8 * 64 * 4;                      // [wave][64]
    float* red_l = red_m + kSplit * 64;                              // [wave][64]
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = o_acc[j >> 2][4 * (j & 3) + e];
        *reinterpret_cast<f32x4*>(red_o + ((wave * 8 + j) * 64 + lane) * 4) = v;
    }
    red_m[wave * 64 + lane] = m_run;
    red_l[wave * 64 + lane] = sum_across_halves(l_run);
    __syncthreads();

    float m_tot = -INFINITY;
#pragma unroll
    for (int w = 0; w < kSplit; ++w) m_tot = fmaxf(m_tot, red_m[w * 64 + lane]);
    float weight[kSplit];
    float l_tot = 0.0f;
#pragma unroll
    for (int w = 0; w < kSplit; ++w) {
        const float m_w = red_m[w * 64 + lane];
        // A wave that saw no keys has m_w = -inf, l_w = 0, O_w = 0: weight 0.
        weight[w] = m_w == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m_w - m_tot) * scale_log2);
        l_tot += red_l[w * 64 + lane] * weight[w];
    }
    const float inv_l = 1.0f / l_tot;
    // The block's FP16 output tile goes through LDS (past the merge area): float group j
    // of row lq is 16-byte chunk j of the row, XOR-swizzled by the row; then the waves
    // store whole 128-byte rows, one 16-byte chunk per lane (32 / kSplit rows per wave).
    uint8_t* const out_lds = smem + kMergeBytes;
#pragma unroll
    for (int j0 = 0; j0 < 8; j0 += kSplit) {
        const int j = j0 + wave;
        if (kSplit < 8 && j >= 8) break;
        f32x4 acc = {};
#pragma unroll
        for (int w = 0; w < kSplit; ++w) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(red_o + ((w * 8 + j) * 64 + lane) * 4);
            acc += v * weight[w];
        }
        // Float j holds dims 32*(j/4) + 8*(j%4) + 4*half + 0..3 of my_query: chunk j, half `half`.
        const f16x2 a = pack_rn(acc[0] * inv_l, acc[1] * inv_l);
        const f16x2 c = pack_rn(acc[2] * inv_l, acc[3] * inv_l);
        *reinterpret_cast<f16x4*>(out_lds + lq * kRowBytes + ((j ^ (lq & 7)) << 4) + 8 * half) =
            __builtin_shufflevector(a, c, 0, 1, 2, 3);
    }
    __syncthreads();
    constexpr int kRowsPerWave = kQueriesPerWave / kSplit;
    if ((lane >> 3) >= kRowsPerWave) return;
    const int out_row = kRowsPerWave * wave + (lane >> 3);
    const int chunk = lane & 7;
    const f16x8 row_chunk = *reinterpret_cast<const f16x8*>(out_lds + out_row * kRowBytes + ((chunk ^ (out_row & 7)) << 4));
    if (kPartial && q0 + out_row >= seq_len) return;
    *reinterpret_cast<f16x8*>(o_head + (size_t)(q0 + out_row) * kHeadDim + 8 * chunk) = row_chunk;
}

// Key-split kernel with dedicated DMA waves. A CU fills its LDS from L2 at about 64 B
// per clock, and a wave that issues LDS-DMA while its earlier DMAs are in flight
// stalls at the issue. In fa2_forward_splitk_kernel each wave fetches its own tiles,
// so while it computes one tile only the next is in flight (64 KiB per CU), and the
// fetch runs at about half that rate. Here kSplit consumer waves only compute and
// kSplit producer waves (producer w + kSplit serves consumer w, on the same SIMD)
// only issue and wait for DMA. Consumer w streams its share of the key tiles through
// two LDS stages of its own: at step j it reads tile j (K, V) into registers and
// releases the stage, and its producer refills the stage with tile j+2, so two tiles
// per consumer are in flight while the consumers compute. Steps are separated by
// two workgroup barriers (X_j: tile j landed, Y_j: tile j read), and every wave runs
// the same number of steps. Q rows are fetched once (by producer 0). The merge of the
// consumers' partial results is that of fa2_forward_splitk_kernel.
template <bool kCausal, bool kPartial, int kSplit, int kBlocks>
__global__ __launch_bounds__(2 * kSplit * 64) void fa2_forward_splitk_dma_waves_kernel(const _Float16* __restrict__ query,
                                                                       const _Float16* __restrict__ key,
                                                                       const _Float16* __restrict__ value,
                                                                       _Float16* __restrict__ output,
                                                                       int seq_len, int num_query_blocks,
                                                                       float scale_log2) {
    constexpr int kTileKeys = 32 * kBlocks;
    constexpr int kTileBytesW = kTileKeys * kRowBytes;
    constexpr int kStageBytes = 2 * kTileBytesW;            // K tile then V tile
    constexpr int kDmaPerMatrix = kTileBytesW / 1024;
    constexpr int kDmaPerTile = 2 * kDmaPerMatrix;
    constexpr int kMergeBytes = kSplit * (8 * 64 * 16 + 2 * 64 * 4);
    constexpr int kQBytes = kQueriesPerWave * kRowBytes;     // one copy of the block's Q rows
    constexpr int kRingBytes = kSplit * 2 * kStageBytes;
    constexpr int kSmemBytes = kRingBytes + kQBytes > kMergeBytes ? kRingBytes + kQBytes : kMergeBytes;
    static_assert(kSplit == 4, "the epilogue stores 8 rows per consumer wave");
    static_assert(kMergeBytes + kQueriesPerWave * kRowBytes <= kSmemBytes, "output tile past the merge area");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kSmemBytes];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool producer = wave >= kSplit;
    const int cw = producer ? wave - kSplit : wave;
    const int lane = tid & 63;
    const int lq = lane & 31;
    const int half = lane >> 5;

    const uint32_t groups = gridDim.x;
    const uint32_t xcd = blockIdx.x & 7u;
    const uint32_t slot = blockIdx.x >> 3;
    const uint32_t per_xcd = groups >> 3;
    const uint32_t extra = groups & 7u;
    const uint32_t logical = xcd * per_xcd + min(xcd, extra) + slot;
    const uint32_t bh = logical / (uint32_t)num_query_blocks;
    uint32_t qblock = logical - bh * (uint32_t)num_query_blocks;
    if (kCausal) qblock = (uint32_t)num_query_blocks - 1u - qblock;

    const size_t head_offset = (size_t)bh * (size_t)seq_len * kHeadDim;
    const _Float16* __restrict__ q_head = query + head_offset;
    _Float16* __restrict__ o_head = output + head_offset;

    const int q0 = (int)qblock * kQueriesPerWave;
    const int my_query = q0 + lq;
    const bool query_valid = !kPartial || my_query < seq_len;
    const int visible_tiles = kCausal ? (q0 + kQueriesPerWave - 1) / kTileKeys + 1
                                      : (seq_len + kTileKeys - 1) / kTileKeys;
    const int t_begin = cw * visible_tiles / kSplit;
    const int t_end = (cw + 1) * visible_tiles / kSplit;
    const int n_tiles = t_end - t_begin;
    const int n_steps = (visible_tiles + kSplit - 1) / kSplit;  // the same for every wave

    uint8_t* const ring = smem + cw * 2 * kStageBytes;
    uint8_t* const q_lds = smem + kRingBytes;

    if (producer) {
        const u32x4 k_head = head_descriptor(key + head_offset, seq_len);
        const u32x4 v_head = head_descriptor(value + head_offset, seq_len);
        const uint32_t ring_addr = lds_address(ring);
        const int dma_off[2] = {dma_lane_offset(lane, 0), dma_lane_offset(lane, 1)};
        auto dma_tile = [&](int t, int st) {
            const bool partial = kPartial && (t + 1) * kTileKeys > seq_len;  // wave-uniform
#pragma unroll
            for (int n = 0; n < kDmaPerTile; ++n) {
                const int m = n / kDmaPerMatrix;
                const int r0 = (n % kDmaPerMatrix) * 8;
                const uint32_t lds = ring_addr + (uint32_t)(st * kStageBytes + m * kTileBytesW + r0 * kRowBytes);
                const int src = t * kTileBytesW + r0 * kRowBytes;
                const int off = dma_off[(r0 >> 3) & 1];
                if (partial) dma16_asm_checked(m ? v_head : k_head, lds, off + src);
                else dma16_asm(m ? v_head : k_head, lds, off, src);
            }
        };
        if (cw == 0) {
            // Rows past seq_len read as zeros (partial block).
            const u32x4 q_desc = head_descriptor(q_head, seq_len);
            const uint32_t q_addr = lds_address(q_lds);
#pragma unroll
            for (int n = 0; n < kQBytes / 1024; ++n) {
                const int r0 = n * 8;
                const int src = (q0 + r0) * kRowBytes;
                if (kPartial) dma16_asm_checked(q_desc, q_addr + (uint32_t)(r0 * kRowBytes), dma_off[n & 1] + src);
                else dma16_asm(q_desc, q_addr + (uint32_t)(r0 * kRowBytes), dma_off[n & 1], src);
            }
        }
        if (n_tiles > 0) dma_tile(t_begin, 0);
        if (n_tiles > 1) dma_tile(t_begin + 1, 1);
        for (int j = 0; j < n_steps; ++j) {
            if (j + 1 < n_tiles) asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kDmaPerTile) : "memory");  // X_j
            else asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
            asm volatile("s_barrier" ::: "memory");  // Y_j
            if (j + 2 < n_tiles) dma_tile(t_begin + j + 2, j & 1);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        __syncthreads();
        __syncthreads();
        return;
    }

    const int q_swz = tile_swizzle(lq);
    f16x8 q_frag[4];
    const int k_row = key_of_mfma_row(lq);
    const int k_swz = tile_swizzle(k_row);
    int k_off[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) k_off[ks] = k_row * kRowBytes + (((2 * ks + half) ^ k_swz) << 4);
    const int grp = lane >> 4;
    const int i16 = lane & 15;
    int v_off[2][2];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int dblk = 0; dblk < 2; ++dblk) {
            const int row = 8 * half + 4 * r + (i16 >> 2);
            const int chunk = 4 * dblk + 2 * (grp & 1) + ((i16 & 3) >> 1);
            v_off[r][dblk] = row * kRowBytes + ((chunk ^ tile_swizzle(row)) << 4) + 8 * (i16 & 1);
        }

    f32x16 o_acc[2];
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
        for (int i = 0; i < 16; ++i) o_acc[d][i] = 0.0f;
    float m_run = -INFINITY;
    float l_run = 0.0f;
    const f16x2 ones = {(_Float16)1.0f, (_Float16)1.0f};

    auto exact_max_update = [&](const f32x16 (&s)[kBlocks]) -> bool {
        float tile_max = -INFINITY;
#pragma unroll
        for (int b = 0; b < kBlocks; ++b)
#pragma unroll
            for (int i = 0; i < 16; i += 2) tile_max = fmaxf(fmaxf(tile_max, s[b][i]), s[b][i + 1]);
        tile_max = max_across_halves(tile_max);
        const bool grow = tile_max * scale_log2 > m_run * scale_log2 + kRescaleLog2;
        if (__builtin_amdgcn_ballot_w64(grow) == 0) return false;
        const float m_new = fmaxf(m_run, tile_max);
        const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * scale_log2);
        l_run *= alpha;
#pragma unroll
        for (int d = 0; d < 2; ++d)
#pragma unroll
            for (int i = 0; i < 16; ++i) o_acc[d][i] *= alpha;
        m_run = m_new;
        return true;
    };
    auto tile_probs = [&](const f32x16 (&s)[kBlocks], f16x8 (&pf)[kBlocks][2]) -> float {
        const float m_scaled = m_run * scale_log2;
        float sum = 0.0f;
#pragma unroll
        for (int b = 0; b < kBlocks; ++b) {
            f16x2 pk[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                pk[q] = pack_rn(__builtin_amdgcn_exp2f(fmaf(s[b][2 * q], scale_log2, -m_scaled)),
                                __builtin_amdgcn_exp2f(fmaf(s[b][2 * q + 1], scale_log2, -m_scaled)));
                if (q & 1) sum = __builtin_amdgcn_fdot2(pk[q - 1] + pk[q], ones, sum, false);
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const f16x4 lo = __builtin_shufflevector(pk[4 * h], pk[4 * h + 1], 0, 1, 2, 3);
                const f16x4 hi = __builtin_shufflevector(pk[4 * h + 2], pk[4 * h + 3], 0, 1, 2, 3);
                pf[b][h] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
            }
        }
        return sum;
    };

    for (int j = 0; j < n_steps; ++j) {
        asm volatile("s_barrier" ::: "memory");  // X_j: tile j landed
        const bool active = j < n_tiles;
        const uint8_t* k_lds = ring + (j & 1) * kStageBytes;
        const uint8_t* v_lds = k_lds + kTileBytesW;
        f16x8 kf[kBlocks][4];
        f16x8 vf[4 * kBlocks];
        if (active) {
            if (j == 0) {
#pragma unroll
                for (int ks = 0; ks < 4; ++ks)
                    q_frag[ks] = *reinterpret_cast<const f16x8*>(q_lds + lq * kRowBytes + (((2 * ks + half) ^ q_swz) << 4));
            }
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int b = 0; b < kBlocks; ++b)
                    kf[b][ks] = *reinterpret_cast<const f16x8*>(k_lds + b * 32 * kRowBytes + k_off[ks]);
#pragma unroll
            for (int k = 0; k < 4 * kBlocks; ++k) {
                const int row_base = (32 * (k >> 2) + 16 * ((k >> 1) & 1)) * kRowBytes;
                const f16x4 v_lo = lds_read_transposed(v_lds + row_base + v_off[0][k & 1]);
                const f16x4 v_hi = lds_read_transposed(v_lds + row_base + v_off[1][k & 1]);
                vf[k] = __builtin_shufflevector(v_lo, v_hi, 0, 1, 2, 3, 4, 5, 6, 7);
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // Y_j: stage j & 1 free
        if (active) {
            const int t = t_begin + j;
            f32x16 sc[kBlocks];
            const f32x16 zero = {};
#pragma unroll
            for (int b = 0; b < kBlocks; ++b) sc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[b][0], q_frag[0], zero, 0, 0, 0);
#pragma unroll
            for (int ks = 1; ks < 4; ++ks)
#pragma unroll
                for (int b = 0; b < kBlocks; ++b)
                    sc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[b][ks], q_frag[ks], sc[b], 0, 0, 0);
            const bool causal_tile = kCausal && t * kTileKeys + kTileKeys - 1 > q0;
            if (causal_tile || (kPartial && (t + 1) * kTileKeys > seq_len)) {
#pragma unroll
                for (int b = 0; b < kBlocks; ++b)
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int key_index = t * kTileKeys + 32 * b + 16 * (i >> 3) + 8 * half + (i & 7);
                        if ((kCausal && key_index > my_query) || (kPartial && key_index >= seq_len))
                            sc[b][i] = -INFINITY;
                    }
            }
            f16x8 pf[kBlocks][2];
            const bool first = j == 0;
            if (first) exact_max_update(sc);
            float tile_sum = tile_probs(sc, pf);
            if (!first && __builtin_amdgcn_ballot_w64(tile_sum > kTileSumBound) != 0) {
                if (exact_max_update(sc)) tile_sum = tile_probs(sc, pf);
            }
            l_run += tile_sum;
#pragma unroll
            for (int k = 0; k < 4 * kBlocks; ++k)
                o_acc[k & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[k], pf[k >> 2][(k >> 1) & 1], o_acc[k & 1], 0, 0, 0);
        }
    }

    // Merge the consumers' partial results (the producers have waited for every DMA).
    __syncthreads();
    float* red_o = reinterpret_cast<float*>(smem);                  // [wave][8][64 lanes][4]
    float* red_m = red_o + kSplit * 8 * 64 * 4;                      // [wave][64]
    float* red_l = red_m + kSplit * 64;                              // [wave][64]
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = o_acc[j >> 2][4 * (j & 3) + e];
        *reinterpret_cast<f32x4*>(red_o + ((cw * 8 + j) * 64 + lane) * 4) = v;
    }
    red_m[cw * 64 + lane] = m_run;
    red_l[cw * 64 + lane] = sum_across_halves(l_run);
    __syncthreads();

    float m_tot = -INFINITY;
#pragma unroll
    for (int w = 0; w < kSplit; ++w) m_tot = fmaxf(m_tot, red_m[w * 64 + lane]);
    float weight[kSplit];
    float l_tot = 0.0f;
#pragma unroll
    for (int w = 0; w < kSplit; ++w) {
        const float m_w = red_m[w * 64 + lane];
        weight[w] = m_w == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m_w - m_tot) * scale_log2);
        l_tot += red_l[w * 64 + lane] * weight[w];
    }
    const float inv_l = 1.0f / l_tot;
    // The block's FP16 output tile goes through LDS (past the merge area): float group j
    // of row lq is 16-byte chunk j of the row, XOR-swizzled by the row; then wave w
    // stores rows 8w..8w+7 as whole 128-byte rows, one 16-byte chunk per lane.
    uint8_t* const out_lds = smem + kMergeBytes;
#pragma unroll
    for (int j0 = 0; j0 < 8; j0 += kSplit) {
        const int j = j0 + cw;
        if (kSplit < 8 && j >= 8) break;
        f32x4 acc = {};
#pragma unroll
        for (int w = 0; w < kSplit; ++w) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(red_o + ((w * 8 + j) * 64 + lane) * 4);
            acc += v * weight[w];
        }
        // Float j holds dims 32*(j/4) + 8*(j%4) + 4*half + 0..3 of my_query: chunk j, half `half`.
        const f16x2 a = pack_rn(acc[0] * inv_l, acc[1] * inv_l);
        const f16x2 c = pack_rn(acc[2] * inv_l, acc[3] * inv_l);
        *reinterpret_cast<f16x4*>(out_lds + lq * kRowBytes + ((j ^ (lq & 7)) << 4) + 8 * half) =
            __builtin_shufflevector(a, c, 0, 1, 2, 3);
    }
    __syncthreads();
    const int out_row = 8 * cw + (lane >> 3);
    const int chunk = lane & 7;
    const f16x8 row_chunk = *reinterpret_cast<const f16x8*>(out_lds + out_row * kRowBytes + ((chunk ^ (out_row & 7)) << 4));
    if (kPartial && q0 + out_row >= seq_len) return;
    *reinterpret_cast<f16x8*>(o_head + (size_t)(q0 + out_row) * kHeadDim + 8 * chunk) = row_chunk;
}

// Key order of a 16-key MFMA block in the paired 16-query kernel: group g of 4 rows
// holds keys 4 tau(g) + 0..3, tau = 0, 3, 1, 2 (table in a 16-bit word, 4 bits per entry).
__device__ __forceinline__ int perm16_group(int g) { return (0x2130 >> (4 * g)) & 3; }
__device__ __forceinline__ int perm16(int m) { return 4 * perm16_group(m >> 2) + (m & 3); }
__device__ __forceinline__ int perm16_inverse(int row) { return 4 * ((0x1320 >> (4 * (row >> 2))) & 3) + (row & 3); }

// Max and sum over lanes l, l^16, l^32, l^48: the four lanes that hold one query's
// scores in the 16x16 MFMA layout.
__device__ __forceinline__ float max_across_groups16(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Causal key-split variant with paired 16-query blocks, for causal problems that do
// not fill the chip with 128-query workgroups. In a causal head, query block b
// (16 queries) sees 16(b+1) keys, so one block per workgroup leaves the workgroup of
// the last block with all the keys and the first with a handful. Here a workgroup
// runs block NB-1-p (heavy) and block p (light) of one head (NB = seq_len / 16), so
// every workgroup has the same ceil((NB-p)/4) + ceil((p+1)/4) block-tiles of 64 keys
// (17 at seq_len 1024): half the work of a noncausal 32-query workgroup, in the same
// grid. The light block's tiles are the first of the heavy block's, and each is
// fetched and read from LDS once for both blocks. The workgroup's key tiles are split
// into kSplit contiguous shares, one per wave, balanced by cost (a tile for both blocks
// counts 4, one for the heavy block 3); a wave streams its share through two LDS
// stages of its own, keeps a running max, sum and O per block, and the partial
// results of each block are merged through LDS at the end. Scores come from
// v_mfma_f32_16x16x32_f16 (S^T = K Q^T, 16 keys x 16 queries per MFMA): lane l holds
// query l%16 and four consecutive keys of each 16-key block h (the group l/16 with its
// two bits swapped, times 4, + 0..3: K rows feed the MFMA in that order), so the probabilities
// of a 32-key block are the lane's P^T operand of O^T += V^T P^T as they stand, with
// V^T read by LDS transpose reads.
template <int kSplit>
__global__ __launch_bounds__(kSplit * 64) void fa2_forward_pairs16_kernel(const _Float16* __restrict__ query,
                                                                  const _Float16* __restrict__ key,
                                                                  const _Float16* __restrict__ value,
                                                                  _Float16* __restrict__ output,
                                                                  int seq_len, int pairs_per_head,
                                                                  float scale_log2) {
    constexpr int kBlockQ = 16;
    constexpr int kStageBytes = 2 * kTileBytes;                // K tile then V tile, 16 KiB
    constexpr int kDmaPerTile = kStageBytes / 1024;            // one wave fetches whole tiles
    constexpr int kQBlockBytes = kBlockQ * kRowBytes;          // 2 KiB
    constexpr int kWaveBytes = 2 * kStageBytes + 2 * kQBlockBytes;
    constexpr int kMergeBytes = 2 * kSplit * (64 * 16 * 4 + 2 * 64 * 4);
    constexpr int kSmemBytes = kSplit * kWaveBytes > kMergeBytes ? kSplit * kWaveBytes : kMergeBytes;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kSmemBytes];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int lq = lane & 15;   // query of the block this lane's scores belong to
    const int grp = lane >> 4;  // which 4 keys of each 16 the lane holds

    // Workgroup -> (batch*head, pair), XCD-contiguous.
    const uint32_t groups = gridDim.x;
    const uint32_t xcd = blockIdx.x & 7u;
    const uint32_t slot = blockIdx.x >> 3;
    const uint32_t per_xcd = groups >> 3;
    const uint32_t extra = groups & 7u;
    const uint32_t logical = xcd * per_xcd + min(xcd, extra) + slot;
    const uint32_t bh = logical / (uint32_t)pairs_per_head;
    const int pair = (int)(logical - bh * (uint32_t)pairs_per_head);
    const int blocks_per_head = 2 * pairs_per_head;

    const size_t head_offset = (size_t)bh * (size_t)seq_len * kHeadDim;
    const u32x4 q_desc = head_descriptor(query + head_offset, seq_len);
    const u32x4 k_head = head_descriptor(key + head_offset, seq_len);
    const u32x4 v_head = head_descriptor(value + head_offset, seq_len);
    _Float16* __restrict__ o_head = output + head_offset;

    // Block 0: the heavy block, block 1: the light one. The key tiles of a block are
    // 0..ceil(16(b+1)/64)-1; every tile's first key is at or before the block's first
    // query, so no row of a tile is masked entirely.
    const int q0[2] = {(blocks_per_head - 1 - pair) * kBlockQ, pair * kBlockQ};
    const int tiles0 = (q0[0] + kBlockQ + kKeysPerTile - 1) / kKeysPerTile;
    const int tiles1 = (q0[1] + kBlockQ + kKeysPerTile - 1) / kKeysPerTile;
    // The light block's key tiles 0..tiles1-1 are a subset of the heavy block's
    // 0..tiles0-1: tile i < tiles1 is fetched once and computed for both blocks, the
    // others for the heavy block only. Wave w takes a contiguous range of tiles with about
    // 1/kSplit of the cost, counting a tile for both blocks as 4 and one for the heavy
    // block as 3 (the fetch and K/V reads are shared). Measured on MI355X against the
    // block-tile split (17 items over 4 waves at seq_len 1024): -8% at B1 H8 N1024 and
    // B1 H2 N1024, -4% to -7% at 1280-1920 keys; 4:3 was 2-6% faster than 3:2 from
    // 1280 keys on and equal at 1024.
    const int total_cost = 4 * tiles1 + 3 * (tiles0 - tiles1);
    auto split_at = [&](int w) -> int {
        const int target = (w * total_cost + kSplit / 2) / kSplit;
        return target <= 4 * tiles1 ? (target + 3) / 4 : tiles1 + (target - 4 * tiles1 + 2) / 3;
    };
    const int t_begin = split_at(wave);
    const int t_end = split_at(wave + 1);

    uint8_t* const my_stages = smem + wave * kWaveBytes;
    const uint32_t my_stages_addr = lds_address(my_stages);
    uint8_t* const my_q = my_stages + 2 * kStageBytes;
    const uint32_t my_q_addr = my_stages_addr + 2 * kStageBytes;
    const int dma_off[2] = {dma_lane_offset(lane, 0), dma_lane_offset(lane, 1)};

    // Both blocks' Q rows to this wave's LDS area, ahead of its first key tile, in the
    // order the K rows feed the MFMA (LDS row perm16(j) holds query row j; see below):
    // lane i of the DMA writes LDS row R = 8n + i/8 and so reads query row
    // perm16_inverse(R).
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int n = 0; n < kQBlockBytes / 1024; ++n) {
            const int lds_row = 8 * n + (lane >> 3);
            const int q_lane_off = perm16_inverse(lds_row) * kRowBytes + (((lane & 7) ^ tile_swizzle(lds_row)) << 4);
            dma16_asm(q_desc, my_q_addr + (uint32_t)(b * kQBlockBytes + n * 1024), q_lane_off, q0[b] * kRowBytes);
        }
    auto dma_tile = [&](int t, int st) {
#pragma unroll
        for (int n = 0; n < kDmaPerTile; ++n) {
            const int m = n / 8;
            const int r0 = (n % 8) * 8;
            dma16_asm(m ? v_head : k_head,
                      my_stages_addr + (uint32_t)(st * kStageBytes + m * kTileBytes + r0 * kRowBytes),
                      dma_off[(r0 >> 3) & 1], t * kTileBytes + r0 * kRowBytes);
        }
    };
    if (t_begin < t_end) dma_tile(t_begin, 0);

    // Per-lane LDS offsets. K (A operand of S^T = K Q^T): MFMA row lq of a 16-key block
    // reads key row perm16(lq), dims 32ks + 8grp..+7 (chunk 4ks + grp). perm16 moves
    // whole groups of 4 rows (group g to group tau(g), tau = 0, 3, 1, 2), so lane group
    // grp holds the 4 consecutive keys 4 tau(grp) + 0..3 of each 16 and the V transpose
    // reads stay 4-row reads; the order makes the 8 rows of every K read pass differ
    // in bit 3 and the 8 rows of every V transpose pass differ in bit 2, which the
    // swizzle maps to distinct banks (measured: no bank conflicts at B1 H8 N1024 causal
    // against 149k per launch in natural order). Q (B operand): query lq, stored at LDS
    // row perm16(lq) by the DMA above, so its reads spread the same way.
    const int key_grp = perm16_group(grp);
    const int k_row = perm16(lq);
    const int swz_k = tile_swizzle(k_row);
    int k_off[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) k_off[ks] = k_row * kRowBytes + (((4 * ks + grp) ^ swz_k) << 4);
    const int (&q_off)[2] = k_off;
    // V^T (A operand of O^T += V^T P^T) by transpose reads: in lane group grp, lane lq
    // reads row 4key_grp + lq/4 (plus 16h + 32kb) at dims 16dblk + 4(lq%4)..+3; the read
    // returns to it dim 16dblk + lq at the group's four keys.
    const int v_row = 4 * key_grp + (lq >> 2);
    const int swz_v = tile_swizzle(v_row);
    int v_off[4];
#pragma unroll
    for (int dblk = 0; dblk < 4; ++dblk)
        v_off[dblk] = v_row * kRowBytes + (((2 * dblk + ((lq & 3) >> 1)) ^ swz_v) << 4) + 8 * (lq & 1);

    f32x4 o[2][4];
    float m_run[2] = {-INFINITY, -INFINITY};
    float l_run[2] = {0.0f, 0.0f};
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int d = 0; d < 4; ++d) o[b][d] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    f16x8 qf[2][2];

    // Block b's scores of tile t from the K fragments in registers, softmax, and P.V
    // with the V fragments. S[kb][h]: keys 32kb + 16h + 4key_grp + 0..3, query q0[b] + lq.
    auto block_tile = [&](auto block_tag, int t, bool first, const f16x8 (&kf)[2][2][2], const f16x8 (&vf)[2][4]) {
        constexpr int b = decltype(block_tag)::value;
        f32x4 s[2][2];
        const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                s[kb][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[kb][h][0], qf[b][0], zero, 0, 0, 0);
                s[kb][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[kb][h][1], qf[b][1], s[kb][h], 0, 0, 0);
            }
        // Causal mask on tiles reaching past the block's first query.
        const int my_query = q0[b] + lq;
        if (t * kKeysPerTile + kKeysPerTile - 1 > q0[b]) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (t * kKeysPerTile + 32 * kb + 16 * h + 4 * key_grp + r > my_query) s[kb][h][r] = -INFINITY;
        }
        // Online softmax with the lazy rescale (bound 2^kRescaleLog2): the first tile of
        // a block in the wave's range takes the exact max; later tiles use the running
        // max and check the lane sums, taking the exact max and recomputing only when a
        // sum exceeds it.
        auto exact_max_update = [&]() -> bool {
            float tile_max = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    tile_max = fmaxf(fmaxf(fmaxf(tile_max, s[kb][h][0]), fmaxf(s[kb][h][1], s[kb][h][2])), s[kb][h][3]);
            tile_max = max_across_groups16(tile_max);
            const bool grow = tile_max * scale_log2 > m_run[b] * scale_log2 + kRescaleLog2;
            if (__builtin_amdgcn_ballot_w64(grow) == 0) return false;
            const float m_new = fmaxf(m_run[b], tile_max);
            const float alpha = __builtin_amdgcn_exp2f((m_run[b] - m_new) * scale_log2);
            l_run[b] *= alpha;
#pragma unroll
            for (int d = 0; d < 4; ++d) o[b][d] *= alpha;
            m_run[b] = m_new;
            return true;
        };
        // FP16 P^T operands of the two 32-key blocks and the lane's FP32 sum of the
        // unrounded probabilities.
        f16x8 pf[2];
        auto probs = [&]() -> float {
            const float m_scaled = m_run[b] * scale_log2;
            float part[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                float e[2][4];
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        e[h][r] = __builtin_amdgcn_exp2f(fmaf(s[kb][h][r], scale_log2, -m_scaled));
                const f16x4 lo = __builtin_shufflevector(pack_rn(e[0][0], e[0][1]), pack_rn(e[0][2], e[0][3]), 0, 1, 2, 3);
                const f16x4 hi = __builtin_shufflevector(pack_rn(e[1][0], e[1][1]), pack_rn(e[1][2], e[1][3]), 0, 1, 2, 3);
                pf[kb] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                part[kb] = ((e[0][0] + e[0][1]) + (e[0][2] + e[0][3])) + ((e[1][0] + e[1][1]) + (e[1][2] + e[1][3]));
            }
            return part[0] + part[1];
        };
        if (first) exact_max_update();
        float tile_sum = probs();
        if (!first && __builtin_amdgcn_ballot_w64(tile_sum > kTileSumBound) != 0) {
            if (exact_max_update()) tile_sum = probs();
        }
        l_run[b] += tile_sum;
        // O^T += V^T P^T for the two 32-key blocks and the four 16-dim blocks.
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int dblk = 0; dblk < 4; ++dblk)
                o[b][dblk] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[kb][dblk], pf[kb], o[b][dblk], 0, 0, 0);
    };

    for (int t = t_begin; t < t_end; ++t) {
        const int st = (t - t_begin) & 1;
        if (t + 1 < t_end) {
            dma_tile(t + 1, st ^ 1);
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kDmaPerTile) : "memory");  // tile t (and Q) landed
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        const bool first = t == t_begin;
        const bool both = t < tiles1;
        if (first) {
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int ks = 0; ks < 2; ++ks)
                    qf[b][ks] = *reinterpret_cast<const f16x8*>(my_q + b * kQBlockBytes + q_off[ks]);
        }
        const uint8_t* k_lds = my_stages + st * kStageBytes;
        const uint8_t* v_lds = k_lds + kTileBytes;
        f16x8 kf[2][2][2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint8_t* rows = k_lds + (32 * kb + 16 * h) * kRowBytes;
                kf[kb][h][0] = *reinterpret_cast<const f16x8*>(rows + k_off[0]);
                kf[kb][h][1] = *reinterpret_cast<const f16x8*>(rows + k_off[1]);
            }
        f16x8 vf[2][4];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int dblk = 0; dblk < 4; ++dblk) {
                const f16x4 lo = lds_read_transposed(v_lds + (32 * kb) * kRowBytes + v_off[dblk]);
                const f16x4 hi = lds_read_transposed(v_lds + (32 * kb + 16) * kRowBytes + v_off[dblk]);
                vf[kb][dblk] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
            }
        block_tile(std::integral_constant<int, 0>{}, t, first, kf, vf);
        if (both) block_tile(std::integral_constant<int, 1>{}, t, first, kf, vf);
    }

    // Merge the partial results of each block (stages are free once every wave is done;
    // a wave without tiles still has its Q DMA to wait for).
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    f32x4* red_o = reinterpret_cast<f32x4*>(smem);                    // [block][wave][dblk][lane]
    float* red_m = reinterpret_cast<float*>(red_o + 2 * kSplit * 4 * 64);  // [block][wave][lane]
    float* red_l = red_m + 2 * kSplit * 64;                              // [block][wave][lane]
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
        for (int d = 0; d < 4; ++d) red_o[((b * kSplit + wave) * 4 + d) * 64 + lane] = o[b][d];
        red_m[(b * kSplit + wave) * 64 + lane] = m_run[b];
        red_l[(b * kSplit + wave) * 64 + lane] = l_run[b];
    }
    __syncthreads();

    // Wave w finishes block (2w / kSplit), 16-dim blocks dblk of a share of the four.
    constexpr int kDblkPerWave = 8 / kSplit;  // 2 with 4 waves, 1 with 8
    const int b = 2 * wave / kSplit;
    const int dblk0 = (wave % (kSplit / 2)) * kDblkPerWave;
    float m_tot = -INFINITY;
#pragma unroll
    for (int w = 0; w < kSplit; ++w) m_tot = fmaxf(m_tot, red_m[(b * kSplit + w) * 64 + lane]);
    float weight[kSplit];
    float l_tot = 0.0f;
#pragma unroll
    for (int w = 0; w < kSplit; ++w) {
        const float m_w = red_m[(b * kSplit + w) * 64 + lane];
        // A wave that saw no keys of this block has m_w = -inf, l_w = 0, O_w = 0: weight 0.
        weight[w] = m_w == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m_w - m_tot) * scale_log2);
        float l_w = 0.0f;
#pragma unroll
        for (int g = 0; g < 4; ++g) l_w += red_l[(b * kSplit + w) * 64 + 16 * g + lq];
        l_tot += l_w * weight[w];
    }
    const float inv_l = 1.0f / l_tot;
    // Both blocks' FP16 output rows go through LDS (past the merge area): row lq of block
    // b, 16-byte chunk c at (c ^ (row & 7)); then wave w stores 32 / kSplit whole rows.
    uint8_t* const out_lds = smem + kMergeBytes;
#pragma unroll
    for (int x = 0; x < kDblkPerWave; ++x) {
        const int dblk = dblk0 + x;
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int w = 0; w < kSplit; ++w) acc += red_o[((b * kSplit + w) * 4 + dblk) * 64 + lane] * weight[w];
        // Lane holds dims 16dblk + 4grp + 0..3 of query q0 + lq: chunk 2dblk + grp/2, half grp%2.
        const f16x2 lo = pack_rn(acc[0] * inv_l, acc[1] * inv_l);
        const f16x2 hi = pack_rn(acc[2] * inv_l, acc[3] * inv_l);
        const int row = 16 * b + lq;
        *reinterpret_cast<f16x4*>(out_lds + row * kRowBytes + (((2 * dblk + (grp >> 1)) ^ (row & 7)) << 4) + 8 * (grp & 1)) =
            __builtin_shufflevector(lo, hi, 0, 1, 2, 3);
    }
    __syncthreads();
    constexpr int kRowsPerWave = 32 / kSplit;
    if ((lane >> 3) >= kRowsPerWave) return;
    const int out_row = kRowsPerWave * wave + (lane >> 3);  // 0..15 block 0, 16..31 block 1
    const int chunk = lane & 7;
    const f16x8 row_chunk = *reinterpret_cast<const f16x8*>(out_lds + out_row * kRowBytes + ((chunk ^ (out_row & 7)) << 4));
    *reinterpret_cast<f16x8*>(o_head + (size_t)(q0[out_row >> 4] + (out_row & 15)) * kHeadDim + 8 * chunk) = row_chunk;
}

// Wide variant: 64 queries per wave, as two 32-query blocks a and b that share every
// K and V^T fragment - each fragment read from LDS feeds two MFMAs - so LDS reads
// and K/V fetches per FLOP are half those of the 32-query kernel. With random data
// the chip runs at its power limit, and the saved LDS traffic buys clock. Four
// waves (256 queries, blocks 0..7) per workgroup, two workgroups per CU. A tile is
// three phases per wave (K reads and 16 score MFMAs; V^T reads and the softmax of
// both blocks; 16 P.V MFMAs); the two waves of a SIMD, from different workgroups,
// overlap one another's MFMA and softmax phases. LDS: four 16 KiB stages (K then
// V), tile t in stage t % 4, fetched three tiles ahead by LDS-DMA (inline assembly:
// the compiler adds no waits for it; the loop waits with explicit vmcnt) with one
// barrier per tile.
//
// Blocks of a wave: noncausal, 2w and 2w+1. Causal, w and 7-w: block j's last key
// tile is the workgroup's first diagonal tile + j/2, so with adjacent blocks wave 3
// computes two blocks in each of the four diagonal tiles while wave 0 idles in three;
// paired this way the waves' work there is 2, 2, 1 and 1 blocks per tile, and the
// workgroup's tile chain is two block-tiles shorter. Measured on MI355X (same
// process, bit-identical): -5.6% at B16 H16 N4096, -9% at B16 H16 N2048, -7% at
// B16 H16 N1024, -1.7% at B2 H32 N16384.
//
// Causal schedules (kPairs):
//  - false: one query tile per workgroup. Each XCD takes its own heads a group at a
//    time, and within a group the query tiles run heaviest first across all its
//    heads (every head's last tile, then every head's second-to-last, ...). A group
//    has about as many tiles as an XCD has workgroup slots (64: 32 CUs, two
//    workgroups each), so its workgroups start on the same keys together and its
//    heads' K/V is read from HBM about once and shared through L2; the
//    longest-first order drains the workgroup slots of the chip evenly.
//  - true: a workgroup runs query tile T-1-p and then tile p of one head (T even),
//    so every workgroup streams the same 4(T+1) key tiles: better when the grid is
//    only one or two rounds of workgroups, where the group order has too few tiles
//    to balance; the light pass re-reads keys that have left L2.
// Heads per group for T query tiles per head (group_heads): 64 / T, from 1 to 8. Measured on
// MI355X (same process): at T = 16 (B16 H16 N4096) groups of 4 fetch 1.04x Q+K+V from HBM
// against 1.69x for groups of 8; at T = 64 (B2 H32 N16384) one head per group fetches 1.13x
// against 6.9x for 8. With the balanced wave blocks and the level order, 128 / T heads per
// group ran between 4% faster and 1% slower than 64 / T on two boxes (B16 H16 N4096, B2 H16
// N8192, B4 H16 N2048, B2 H32 N16384, B64 H16 N512), and 256 / T up to 2% slower.

// Softmax helpers of the kernels that hold one 32-query block's 64-key tile of scores as two
// 32x32 accumulators s[0], s[1] (S^T: the lane's query column; register i of key block kb
// holds key 64t + 32kb + 16(i/8) + 8*half + i%8). The running max is kept scaled,
// mc = max * scale_log2 (log2 units), so a probability is exp2(s * scale_log2 - mc): one FMA,
// with no per-tile product of the max.
// Exact tile max and lazy rescale of l and O (bound 2^kRescaleLog2); returns whether the
// max moved. The rescale factor exp2(mc_old - mc_new) is the exact ratio between the
// probabilities formed against the two maxima.
__device__ __forceinline__ bool block_exact_max_update(const f32x16 (&s)[2], float scale_log2, float& mc_run,
                                                       float& l_run, f32x16 (&o)[2]) {
    float tile_max = -INFINITY;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int i = 0; i < 16; i += 2) tile_max = fmaxf(fmaxf(tile_max, s[b][i]), s[b][i + 1]);
    const float tile_mc = max_across_halves(tile_max) * scale_log2;
    const bool grow = tile_mc > mc_run + kRescaleLog2;
    if (__builtin_amdgcn_ballot_w64(grow) == 0) return false;
    const float mc_new = fmaxf(mc_run, tile_mc);
    const float alpha = __builtin_amdgcn_exp2f(mc_run - mc_new);
    l_run *= alpha;
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[d][i] *= alpha;
    mc_run = mc_new;
    return true;
}

// FP16 probabilities of the block against its scaled running max, as P.V B operands
// (pf[key block][16-key half]); returns the lane sum (pairs added in FP16, then v_dot2
// against 1.0 into FP32).
__device__ __forceinline__ float block_tile_probs(const f32x16 (&s)[2], float mc_run, float scale_log2,
                                                  f16x8 (&pf)[2][2]) {
    const f16x2 ones = {(_Float16)1.0f, (_Float16)1.0f};
    float sum = 0.0f;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        f16x2 pk[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            pk[q] = pack_rn(__builtin_amdgcn_exp2f(fmaf(s[b][2 * q], scale_log2, -mc_run)),
                            __builtin_amdgcn_exp2f(fmaf(s[b][2 * q + 1], scale_log2, -mc_run)));
            if (q & 1) sum = __builtin_amdgcn_fdot2(pk[q - 1] + pk[q], ones, sum, false);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const f16x4 lo = __builtin_shufflevector(pk[4 * h], pk[4 * h + 1], 0, 1, 2, 3);
            const f16x4 hi = __builtin_shufflevector(pk[4 * h + 2], pk[4 * h + 3], 0, 1, 2, 3);
            pf[b][h] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        }
    }
    return sum;
}

// Scores of key tile t past the lane's `query` set to -inf. The sign of limit - offset
// selects -inf by bit select: compares would be hoisted out of the key loop as 64 lane
// masks in SGPRs, and spill. Per 8-key group one opaque base, so that every other constant
// is an inline operand (0..7) rather than an SGPR.
__device__ __forceinline__ void block_mask_diagonal(f32x16 (&s)[2], int query, int t, int half) {
    const int limit = query - t * kKeysPerTile - 8 * half;
    constexpr uint32_t kNegInf = 0xff800000u;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int hi = 0; hi < 2; ++hi) {
            int base = limit - (32 * kb + 16 * hi);
            asm volatile("" : "+v"(base));
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = 8 * hi + j;
                const uint32_t mask = (uint32_t)((base - j) >> 31);
                s[kb][i] = __uint_as_float((mask & kNegInf) | (~mask & __float_as_uint(s[kb][i])));
            }
        }
}

template <bool kCausal, bool kPairs>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void fa2_forward_d64_wide_kernel(const _Float16* __restrict__ query,
                                 const _Float16* __restrict__ key,
                                 const _Float16* __restrict__ value,
                                 _Float16* __restrict__ output,
                                 int seq_len, int num_query_tiles, float scale_log2) {
    constexpr int kWaves = 4;
    constexpr int kWaveQueries = 2 * kQueriesPerWave;
    constexpr int kBlockM = kWaves * kWaveQueries;
    constexpr int kStages = 4;
    constexpr int kStageBytes = 2 * kTileBytes;
    constexpr int kDmaPerTile = kStageBytes / 1024 / kWaves;  // LDS-DMA instructions per wave
    // Causal tile pairs: the last key tile of a pass gets a fifth stage of its own, so that
    // the four diagonal tiles are in LDS together and the waves run them without barriers
    // (80 KiB: still two workgroups per CU). Measured on MI355X (same process, graph replays,
    // bit-identical outputs): -2.6% to -5% at B16 H16 N1024, B8 H64 N1024 and B16 H16 N2048.
    // The head groups keep a barrier per tile: there the last tile fetched with the prologue
    // gained 1% but raised HBM fetch from 1.03x to 1.15x Q+K+V at B16 H16 N4096 (its tile is
    // fetched apart from the head's other workgroups), and fetched two tiles before the
    // diagonal it gained nothing (fetch 1.08x).
    constexpr bool kFreeDiag = kCausal && kPairs;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[(kStages + (kFreeDiag ? 1 : 0)) * kStageBytes];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int lq = lane & 31;
    const int half = lane >> 5;

    // Workgroup -> (batch*head, work item), XCD-contiguous. Noncausal: an item is one
    // query tile. Causal: see the schedules above (head groups, or pairs head by head);
    // `item` counts from the heaviest tile (item 0 = tile T-1).
    static_assert(kCausal || !kPairs, "pairs are a causal schedule");
    const uint32_t tiles_per_head = (uint32_t)num_query_tiles;
    const WorkItem work = xcd_work_item<kCausal && !kPairs>(kPairs ? tiles_per_head / 2u : tiles_per_head);
    const uint32_t bh = work.bh;
    const uint32_t item = work.item;
    constexpr int passes = kPairs ? 2 : 1;

    // Q and O of the head through buffer descriptors (SGPR base, 32-bit lane offsets):
    // no 64-bit row addresses stay live in VGPRs across the passes.
    const size_t head_offset = (size_t)bh * (size_t)seq_len * kHeadDim;
    const __amdgpu_buffer_rsrc_t q_head = head_resource(query + head_offset, seq_len);
    const u32x4 k_head = head_descriptor(key + head_offset, seq_len);
    const u32x4 v_head = head_descriptor(value + head_offset, seq_len);
    const __amdgpu_buffer_rsrc_t o_head = head_resource(output + head_offset, seq_len);

    const uint32_t smem_addr = lds_address(smem);
    const int dma_off[2] = {dma_lane_offset(lane, 0), dma_lane_offset(lane, 1)};
    // This wave issues instructions n = wave + x * kWaves of a tile's 16 (8 per
    // matrix, 8 rows each), into ring stage t % 4 or the named stage.
    auto dma_tile = [&](int t, int stage_index = -1) {
        if (stage_index < 0) stage_index = t & (kStages - 1);
        const uint32_t stage = smem_addr + (uint32_t)(stage_index * kStageBytes);
#pragma unroll
        for (int x = 0; x < kDmaPerTile; ++x) {
            const int n = wave + x * kWaves;
            const int m = n >> 3;
            const int r0 = (n & 7) * 8;
            dma16_asm(m ? v_head : k_head, stage + (uint32_t)(m * kTileBytes + r0 * kRowBytes), dma_off[n & 1],
                      t * kTileBytes + r0 * kRowBytes);
        }
    };

    // LDS addresses of the lane's K fragments in stage 0 (stage s is kStageBytes * s
    // further; the second 32-key block 4 KiB further). Kept whole in VGPRs, so that a
    // fragment address is one add of the stage offset per 16-dim step.
    const int k_row = key_of_mfma_row(lq);
    const int k_swz = tile_swizzle(k_row);
    uint32_t k_addr[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        k_addr[ks] = smem_addr + (uint32_t)(k_row * kRowBytes + (((2 * ks + half) ^ k_swz) << 4));
        asm volatile("" : "+v"(k_addr[ks]));
    }
    // K fragments of the tile in LDS stage `stage_index`: kf[key block][16-dim step].
    auto read_k = [&](int stage_index, f16x8 (&kf)[2][4]) {
        const uint32_t stage_off = (uint32_t)(stage_index * kStageBytes);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const FA2_LDS f16x8* frag = reinterpret_cast<const FA2_LDS f16x8*>((size_t)(k_addr[ks] + stage_off));
#pragma unroll
            for (int b = 0; b < 2; ++b) kf[b][ks] = frag[b * 32 * kRowBytes / 16];
        }
    };
    const int grp = lane >> 4;
    const int i16 = lane & 15;
    int v_off[2][2];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int dblk = 0; dblk < 2; ++dblk) {
            const int row = 8 * half + 4 * r + (i16 >> 2);
            const int chunk = 4 * dblk + 2 * (grp & 1) + ((i16 & 3) >> 1);
            v_off[r][dblk] = row * kRowBytes + ((chunk ^ tile_swizzle(row)) << 4) + 8 * (i16 & 1);
        }



    // Epilogue of a pass: O = O^T / l. Accumulator i of d-block dblk holds dim
    // 32*dblk + 8*(i/4) + 4*half + i%4 of the lane's query.
    // Staged through this wave's 4 KiB of stage 3 (free after the last tile's barrier; the
    // next pass's prologue fetches into stages 0..2; with the fifth stage no diagonal tile is
    // in stage 3, which is free from the barrier after the last tile before the diagonal):
    // chunk c of row r at c ^ (r & 7).
    auto store = [&](const f32x16 (&o)[2], float l_run, int q) {
        const float inv_l = 1.0f / sum_across_halves(l_run);
        // The lane index recomputed here, so that nothing but the accumulators stays live
        // across the key loop for this epilogue (the causal kernels use all 256 VGPRs).
        int lane_o = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
        asm volatile("" : "+v"(lane_o));
        const int lq = lane_o & 31, half = lane_o >> 5;
        uint8_t* const out_lds = smem + 3 * kStageBytes + wave * 4096;
#pragma unroll
        for (int dblk = 0; dblk < 2; ++dblk)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f16x2 a = pack_rn(o[dblk][4 * g + 0] * inv_l, o[dblk][4 * g + 1] * inv_l);
                const f16x2 c = pack_rn(o[dblk][4 * g + 2] * inv_l, o[dblk][4 * g + 3] * inv_l);
                const int chunk = 4 * dblk + g;
                *reinterpret_cast<f16x4*>(out_lds + lq * kRowBytes + ((chunk ^ (lq & 7)) << 4) + 8 * half) =
                    __builtin_shufflevector(a, c, 0, 1, 2, 3);
            }
        const int q_row0 = q - lq;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 8 * r + (lane_o >> 3);
            const int chunk = lane_o & 7;
            const f16x8 v = *reinterpret_cast<const f16x8*>(out_lds + row * kRowBytes + ((chunk ^ (row & 7)) << 4));
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), o_head, (q_row0 + row) * kRowBytes + 16 * chunk, 0, 0);
        }
    };

#pragma unroll
    for (int pass = 0; pass < passes; ++pass) {
        const uint32_t qtile = !kCausal ? item : pass == 0 ? (uint32_t)num_query_tiles - 1u - item : item;
        const int q_block = (int)qtile * kBlockM;
        // 32-query blocks a and b of the wave. Noncausal: blocks 2w and 2w+1. Causal:
        // blocks w and 7-w, so that every wave carries the same number of block-tiles in
        // the tile's four diagonal key tiles (block j ends at key tile q_block/64 + j/2).
        const int block_a = kCausal ? wave : 2 * wave;
        const int block_b = kCausal ? 7 - wave : 2 * wave + 1;
        const int query_a = q_block + kQueriesPerWave * block_a + lq;
        const int query_b = q_block + kQueriesPerWave * block_b + lq;
        const int num_tiles = kCausal ? (q_block + kBlockM - 1) / kKeysPerTile + 1 : seq_len / kKeysPerTile;
        // Causal: the last key tile of each block holds its diagonal.
        const int last_a = kCausal ? (q_block + kQueriesPerWave * block_a) / kKeysPerTile : num_tiles - 1;
        const int last_b = kCausal ? (q_block + kQueriesPerWave * block_b) / kKeysPerTile : num_tiles - 1;

        // Q^T fragments of both blocks (B operands of K Q^T). Tiles 0..2 go to stages
        // 0..2 (and with four key tiles the last to stage 4): the previous pass has no fetch
        // in flight, and its waves ran its diagonal tiles without barriers, so every wave
        // first waits here for the others to be done with them.
        f16x8 qa[4], qb[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            qa[ks] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(q_head, query_a * kRowBytes + 32 * ks + 16 * half, 0, 0));
            qb[ks] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(q_head, query_b * kRowBytes + 32 * ks + 16 * half, 0, 0));
        }
        if (kPairs && pass > 0) __builtin_amdgcn_s_barrier();
        dma_tile(0);
        dma_tile(1);  // num_tiles >= 4: seq_len and the causal key range are multiples of 256
        dma_tile(2);
        if (kFreeDiag && num_tiles == 4) dma_tile(3, kStages);  // the last diagonal tile

        f32x16 oa[2], ob[2];
#pragma unroll
        for (int d = 0; d < 2; ++d)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                oa[d][i] = 0.0f;
                ob[d][i] = 0.0f;
            }
        float mc_a = -INFINITY, mc_b = -INFINITY;  // running max per block, times scale_log2
        float l_a = 0.0f, l_b = 0.0f;            // this lane's share of each denominator

        // Prologue: tiles 0..2 and Q landed. The empty asm consumes Q where the compiler
        // adds its own wait for the Q loads: already satisfied here, whereas at the first
        // MFMA its count would also cover the tile-3 fetch issued in between.
        wait_dma_and_barrier<0>();
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) asm volatile("" ::"v"(qa[ks]), "v"(qb[ks]));


        // One key tile: fetch three ahead, and after the work, wait for tile t+1 (only the
        // fetches of the tiles after it may stay in flight) at a barrier, after which
        // every wave is done with tile t's stage.
        // kFreeDiag: the ring carries tiles 0..num_tiles-2, and the last tile goes to stage 4
        // with the fetch two tiles before the diagonal (d = num_tiles - 4), near the other
        // fetches of the same keys (measured 1-3% faster than with the prologue's fetches at
        // B16 H16 N1024, B8 H64 N1024 and B16 H16 N2048). The barrier after the last tile
        // before the diagonal waits for every fetch, and the four diagonal tiles pass no
        // barrier: each wave runs its own (both blocks up to block a's diagonal tile, then
        // block b alone), 5 block-tiles per wave where a barrier per tile made 6.
        auto fetch_ahead = [&](int t) {
            if (t + 3 < num_tiles - (kFreeDiag ? 1 : 0)) dma_tile(t + 3);  // into the stage tile t-1 used
            if (kFreeDiag && t + 6 == num_tiles) dma_tile(num_tiles - 1, kStages);
        };
        auto tile_done = [&](int t) {
            if constexpr (kFreeDiag) {
                if (t + 6 < num_tiles) wait_dma_and_barrier<2 * kDmaPerTile>();
                else if (t + 6 == num_tiles) wait_dma_and_barrier<3 * kDmaPerTile>();  // d, d+1, d+3 in flight
                else if (t + 5 == num_tiles) wait_dma_and_barrier<0>();
            } else {
                if (t + 3 < num_tiles) wait_dma_and_barrier<2 * kDmaPerTile>();
                else if (t + 2 < num_tiles) wait_dma_and_barrier<kDmaPerTile>();
                else wait_dma_and_barrier<0>();
            }
        };
        auto stage_of = [&](int t) { return kFreeDiag && t == num_tiles - 1 ? kStages : t & (kStages - 1); };
        int t = 0;
        for (; t <= last_a; ++t) {
            fetch_ahead(t);
            const int stage_index = stage_of(t);
            const uint8_t* v_lds = smem + stage_index * kStageBytes + kTileBytes;
            // S^T = K Q^T of both blocks; each K fragment feeds two MFMAs. The MFMA
            // phases run at raised wave priority: when both waves of a SIMD can
            // issue, the one with MFMAs goes first and the other's softmax fills the
            // MFMA shadow. All eight K reads are issued before the first MFMA, and all
            // sixteen V^T reads before the softmax (the scheduling barriers keep the
            // compiler from spreading them over the phases).
            __builtin_amdgcn_s_setprio(1);
            f16x8 kf[2][4];
            read_k(stage_index, kf);
            __builtin_amdgcn_sched_barrier(0);
            f32x16 sa[2], sb[2];
            const f32x16 zero = {};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    sa[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[b][ks], qa[ks], ks == 0 ? zero : sa[b], 0, 0, 0);
                    sb[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[b][ks], qb[ks], ks == 0 ? zero : sb[b], 0, 0, 0);
                }
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(0);
            // V^T fragments of the tile (P.V MFMA k: key block k/4, 16-key half
            // (k/2)%2, d-block k%2), read while the softmax runs.
            f16x8 vf[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int row_base = (32 * (k >> 2) + 16 * ((k >> 1) & 1)) * kRowBytes;
                const f16x4 v_lo = lds_read_transposed(v_lds + row_base + v_off[0][k & 1]);
                const f16x4 v_hi = lds_read_transposed(v_lds + row_base + v_off[1][k & 1]);
                vf[k] = __builtin_shufflevector(v_lo, v_hi, 0, 1, 2, 3, 4, 5, 6, 7);
            }
            __builtin_amdgcn_sched_barrier(0);

            // Causal: block a's diagonal tile. Block b (later queries) sees every key
            // of it.
            if (kCausal && t == last_a) block_mask_diagonal(sa, query_a, t, half);

            // Online softmax per block: exact max on the first tile, then the running
            // max with the lane-sum check (every probability is <= 2^kRescaleLog2 when its lane's
            // sum is), recomputing only a block whose check fails.
            f16x8 pa[2][2], pb[2][2];
            if (t == 0) {
                block_exact_max_update(sa, scale_log2, mc_a, l_a, oa);
                block_exact_max_update(sb, scale_log2, mc_b, l_b, ob);
            }
            float sum_a = block_tile_probs(sa, mc_a, scale_log2, pa);
            float sum_b = block_tile_probs(sb, mc_b, scale_log2, pb);
            if (t != 0) {
                if (__builtin_amdgcn_ballot_w64(sum_a > kTileSumBound) != 0 && block_exact_max_update(sa, scale_log2, mc_a, l_a, oa))
                    sum_a = block_tile_probs(sa, mc_a, scale_log2, pa);
                if (__builtin_amdgcn_ballot_w64(sum_b > kTileSumBound) != 0 && block_exact_max_update(sb, scale_log2, mc_b, l_b, ob))
                    sum_b = block_tile_probs(sb, mc_b, scale_log2, pb);
            }
            l_a += sum_a;
            l_b += sum_b;

            // O^T += V^T P^T for both blocks; each V^T fragment feeds two MFMAs.
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                oa[k & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[k], pa[k >> 2][(k >> 1) & 1], oa[k & 1], 0, 0, 0);
                ob[k & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[k], pb[k >> 2][(k >> 1) & 1], ob[k & 1], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(0);
            tile_done(t);
        }
        if constexpr (kCausal) {
            // Tiles past block a's diagonal: the same three phases for block b alone
            // (t >= 1 here, so its running max is set).
            for (; t <= last_b; ++t) {
                fetch_ahead(t);
                const int stage_index = stage_of(t);
                const uint8_t* v_lds = smem + stage_index * kStageBytes + kTileBytes;
                __builtin_amdgcn_s_setprio(1);
                f16x8 kf[2][4];
                read_k(stage_index, kf);
                __builtin_amdgcn_sched_barrier(0);
                f32x16 sb[2];
                const f32x16 zero = {};
#pragma unroll
                for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                    for (int b = 0; b < 2; ++b)
                        sb[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[b][ks], qb[ks], ks == 0 ? zero : sb[b], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_s_setprio(0);
                f16x8 vf[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const int row_base = (32 * (k >> 2) + 16 * ((k >> 1) & 1)) * kRowBytes;
                    const f16x4 v_lo = lds_read_transposed(v_lds + row_base + v_off[0][k & 1]);
                    const f16x4 v_hi = lds_read_transposed(v_lds + row_base + v_off[1][k & 1]);
                    vf[k] = __builtin_shufflevector(v_lo, v_hi, 0, 1, 2, 3, 4, 5, 6, 7);
                }
                __builtin_amdgcn_sched_barrier(0);
                if (t == last_b) block_mask_diagonal(sb, query_b, t, half);
                f16x8 pb[2][2];
                float sum_b = block_tile_probs(sb, mc_b, scale_log2, pb);
                if (__builtin_amdgcn_ballot_w64(sum_b > kTileSumBound) != 0 && block_exact_max_update(sb, scale_log2, mc_b, l_b, ob))
                    sum_b = block_tile_probs(sb, mc_b, scale_log2, pb);
                l_b += sum_b;
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_s_setprio(1);
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    ob[k & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[k], pb[k >> 2][(k >> 1) & 1], ob[k & 1], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_s_setprio(0);
                tile_done(t);
            }
            // The workgroup's remaining tiles: only the fetches and barriers (none with the
            // fifth stage: nothing left to fetch, and the diagonal passes no barrier).
            for (; !kFreeDiag && t < num_tiles; ++t) {
                fetch_ahead(t);
                tile_done(t);
            }
        }

        store(oa, l_a, query_a);
        store(ob, l_b, query_b);
    }  // pass
}

// Causal problems whose 128-query grid fills the chip's workgroup slots about once,
// with long key streams: a workgroup of 8 waves takes the pair of 128-query tiles
// T-1-p (heavy) and p (light) of one head (T = N/128, even), and the pair's 2T+2 key
// tiles of 64 are split evenly between two groups of 4 waves. Group 0 streams the heavy
// tile's key tiles 0..T; group 1 the light tile's 2p+2, then the heavy tile's remaining
// T-2p-1. Wave w of a group owns queries 32(w%4)..32(w%4)+31 of the tile it serves.
// Each group has a 4-stage ring of its own (64 KiB), and both take T+1 steps with one
// workgroup barrier each, so every wave runs the same barriers. A wave skips the
// compute of a key tile that lies wholly past its queries (the light tile's last one
// for waves 0-1, and group 1's heavy keys for waves 0-1 of the middle pair), and every
// wave that computes a tile has a key in it for each of its queries. At the end group 1
// hands its part of the heavy tile (O, scaled max mc and l per lane) to group 0 through LDS:
//   mc = max(mc0, mc1),  l = l0 2^(mc0 - mc) + l1 2^(mc1 - mc),  O likewise,
// and group 0 stores the merged tile. Both tiles' outputs are staged through LDS (16 KiB
// past the rings, 144 KiB in all) and stored as whole 128-byte rows; measured on MI355X
// (same process, with the K and V^T reads issued ahead of their phases), -1% to -3%
// against 8-byte stores straight from the accumulators. With one workgroup per CU every
// SIMD keeps two waves for the same T+1 steps, where one query tile per workgroup left
// the CU of the heaviest tile running it alone, one wave per SIMD.
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2)))
void fa2_forward_d64_split_pairs_kernel(const _Float16* __restrict__ query,
                                        const _Float16* __restrict__ key,
                                        const _Float16* __restrict__ value,
                                        _Float16* __restrict__ output,
                                        int seq_len, int num_query_tiles, float scale_log2) {
    constexpr int kGroupWaves = 4;
    constexpr int kStages = 4;
    constexpr int kStageBytes = 2 * kTileBytes;
    constexpr int kRingBytes = kStages * kStageBytes;
    constexpr int kDmaPerTile = kStageBytes / 1024 / kGroupWaves;  // LDS-DMA instructions per wave
    constexpr int kHandoffFloats = 34;                             // per lane: O (2 x 16), m, l
    constexpr int kOutBytes = 32 * kRowBytes;                      // one wave's 32 x 64 FP16 output block
    static_assert(kGroupWaves * kHandoffFloats * 64 * 4 <= 2 * kRingBytes, "the handoff fits the rings");
    // Past the two rings: each wave index of a group has one output staging block, used by
    // group 1 for the light tile (mid-loop, while the rings stream) and by group 0 for the
    // heavy tile (after the handoff barrier, when group 1's use is long done).
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * kRingBytes + kGroupWaves * kOutBytes];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int group = wave >> 2;
    const int gw = wave & 3;
    const int lane = tid & 63;
    const int lq = lane & 31;
    const int half = lane >> 5;

    const int T = num_query_tiles;
    const WorkItem work = xcd_work_item<false>((uint32_t)T / 2u);
    const int light = (int)work.item;
    const int heavy = T - 1 - light;
    const int light_tiles = 2 * light + 2;  // 64-key tiles of the light tile
    const int steps = T + 1;                // 64-key tiles per group

    const size_t head_offset = (size_t)work.bh * (size_t)seq_len * kHeadDim;
    const __amdgpu_buffer_rsrc_t q_head = head_resource(query + head_offset, seq_len);
    const u32x4 k_head = head_descriptor(key + head_offset, seq_len);
    const u32x4 v_head = head_descriptor(value + head_offset, seq_len);
    const __amdgpu_buffer_rsrc_t o_head = head_resource(output + head_offset, seq_len);

    // Step s of this group: its key tile, and whether it serves the light tile.
    auto on_light = [&](int s) { return group == 1 && s < light_tiles; };
    auto key_tile = [&](int s) { return (group == 0 || s < light_tiles) ? s : T + 1 + (s - light_tiles); };

    uint8_t* const ring = smem + group * kRingBytes;
    const uint32_t ring_addr = lds_address(ring);
    // n & 1 = gw & 1 for every instruction of the wave: one lane offset.
    const int dma_off = dma_lane_offset(lane, gw & 1);
    // The group's waves issue instructions n = gw + x * 4 of a tile's 16 (8 per
    // matrix, 8 rows each) into stage s % 4 of the group's ring.
    auto dma_step = [&](int s) {
        const int kt = key_tile(s);
        const uint32_t stage = ring_addr + (uint32_t)((s & (kStages - 1)) * kStageBytes);
#pragma unroll
        for (int x = 0; x < kDmaPerTile; ++x) {
            const int n = gw + x * kGroupWaves;
            const int m = n >> 3;
            const int r0 = (n & 7) * 8;
            dma16_asm(m ? v_head : k_head, stage + (uint32_t)(m * kTileBytes + r0 * kRowBytes), dma_off,
                      kt * kTileBytes + r0 * kRowBytes);
        }
    };

    const int k_row = key_of_mfma_row(lq);
    const int k_swz = tile_swizzle(k_row);
    int k_off[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) k_off[ks] = k_row * kRowBytes + (((2 * ks + half) ^ k_swz) << 4);
    const int grp = lane >> 4;
    const int i16 = lane & 15;
    int v_off[2][2];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int dblk = 0; dblk < 2; ++dblk) {
            const int row = 8 * half + 4 * r + (i16 >> 2);
            const int chunk = 4 * dblk + 2 * (grp & 1) + ((i16 & 3) >> 1);
            v_off[r][dblk] = row * kRowBytes + ((chunk ^ tile_swizzle(row)) << 4) + 8 * (i16 & 1);
        }

    // First query of this wave's 32-query block in each tile.
    const int q_heavy = heavy * 128 + gw * kQueriesPerWave;
    const int q_light = light * 128 + gw * kQueriesPerWave;

    // Q^T fragments (B operands of K Q^T): the first tile the group serves, and the
    // heavy tile for group 1's second part.
    f16x8 qf[4], qf_heavy[4];
    const int q_start = group == 0 ? q_heavy : q_light;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        qf[ks] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(q_head, (q_start + lq) * kRowBytes + 32 * ks + 16 * half, 0, 0));
        qf_heavy[ks] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(q_head, (q_heavy + lq) * kRowBytes + 32 * ks + 16 * half, 0, 0));
    }
    dma_step(0);
    dma_step(1);
    dma_step(2);  // steps = T + 1 >= 3

    // O / l of one 32-query block as FP16: accumulator i of d-block dblk holds dim
    // 32*dblk + 8*(i/4) + 4*half + i%4 of the lane's query. Staged through the wave's
    // output block in LDS (chunk c of row r at c ^ (r & 7)) and read back a row per 8
    // lanes, so that every store instruction writes whole 128-byte rows. Waves w and w+4
    // share block w: group 1 uses it for the light tile inside the key loop, group 0
    // after the merge, with workgroup barriers in between; within one use a wave's LDS
    // accesses complete in order, so no barrier of its own.
    uint8_t* const out_lds = smem + 2 * kRingBytes + gw * kOutBytes;
    auto store_block = [&](const f32x16 (&o)[2], float l_lane, int q_first) {
        const float inv_l = 1.0f / sum_across_halves(l_lane);
#pragma unroll
        for (int dblk = 0; dblk < 2; ++dblk)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f16x2 a = pack_rn(o[dblk][4 * g + 0] * inv_l, o[dblk][4 * g + 1] * inv_l);
                const f16x2 c = pack_rn(o[dblk][4 * g + 2] * inv_l, o[dblk][4 * g + 3] * inv_l);
                const int chunk = 4 * dblk + g;
                *reinterpret_cast<f16x4*>(out_lds + lq * kRowBytes + ((chunk ^ (lq & 7)) << 4) + 8 * half) =
                    __builtin_shufflevector(a, c, 0, 1, 2, 3);
            }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 8 * r + (lane >> 3);
            const int chunk = lane & 7;
            const f16x8 v = *reinterpret_cast<const f16x8*>(out_lds + row * kRowBytes + ((chunk ^ (row & 7)) << 4));
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), o_head, (q_first + row) * kRowBytes + 16 * chunk, 0, 0);
        }
    };

    f32x16 o[2];
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[d][i] = 0.0f;
    float mc_run = -INFINITY;  // running max of the scores, times scale_log2
    float l_run = 0.0f;       // this lane's share of the denominator
    bool fresh = true;        // no key tile computed yet for the current query tile

    wait_dma_and_barrier<0>();
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) asm volatile("" ::"v"(qf[ks]), "v"(qf_heavy[ks]));

    for (int s = 0; s < steps; ++s) {
        if (s + 3 < steps) dma_step(s + 3);  // into the stage step s-1 used
        if (group == 1 && s == light_tiles) {
            // The light tile is complete: store it, and start the heavy tile's last keys.
            store_block(o, l_run, q_light);
#pragma unroll
            for (int d = 0; d < 2; ++d)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[d][i] = 0.0f;
            mc_run = -INFINITY;
            l_run = 0.0f;
            fresh = true;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) qf[ks] = qf_heavy[ks];
        }
        const int kt = key_tile(s);
        const int q_first = on_light(s) ? q_light : q_heavy;
        if (kt * kKeysPerTile <= q_first + kQueriesPerWave - 1) {
            const uint8_t* k_lds = ring + (s & (kStages - 1)) * kStageBytes;
            const uint8_t* v_lds = k_lds + kTileBytes;
            __builtin_amdgcn_s_setprio(1);
            f16x8 kf[2][4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int b = 0; b < 2; ++b)
                    kf[b][ks] = *reinterpret_cast<const f16x8*>(k_lds + b * 32 * kRowBytes + k_off[ks]);
            // All K reads before the first MFMA and all V^T reads before the softmax, as
            // in the 256-query kernel.
            __builtin_amdgcn_sched_barrier(0);
            f32x16 sc[2];
            const f32x16 zero = {};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int b = 0; b < 2; ++b)
                    sc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[b][ks], qf[ks], ks == 0 ? zero : sc[b], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(0);
            f16x8 vf[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int row_base = (32 * (k >> 2) + 16 * ((k >> 1) & 1)) * kRowBytes;
                const f16x4 v_lo = lds_read_transposed(v_lds + row_base + v_off[0][k & 1]);
                const f16x4 v_hi = lds_read_transposed(v_lds + row_base + v_off[1][k & 1]);
                vf[k] = __builtin_shufflevector(v_lo, v_hi, 0, 1, 2, 3, 4, 5, 6, 7);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (kt * kKeysPerTile + kKeysPerTile - 1 > q_first) block_mask_diagonal(sc, q_first + lq, kt, half);
            const bool first = fresh;
            fresh = false;
            if (first) block_exact_max_update(sc, scale_log2, mc_run, l_run, o);
            f16x8 pf[2][2];
            float sum = block_tile_probs(sc, mc_run, scale_log2, pf);
            if (!first && __builtin_amdgcn_ballot_w64(sum > kTileSumBound) != 0 && block_exact_max_update(sc, scale_log2, mc_run, l_run, o))
                sum = block_tile_probs(sc, mc_run, scale_log2, pf);
            l_run += sum;
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int k = 0; k < 8; ++k)
                o[k & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[k], pf[k >> 2][(k >> 1) & 1], o[k & 1], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(0);
        }
        // Wait for step s+1's tile (only later fetches may stay in flight); after the
        // barrier every wave is done with step s's stage.
        if (s + 3 < steps) wait_dma_and_barrier<2 * kDmaPerTile>();
        else if (s + 2 < steps) wait_dma_and_barrier<kDmaPerTile>();
        else wait_dma_and_barrier<0>();
    }

    // Every wave is past the last step's barrier with no fetch in flight: the rings
    // are free for the handoff (per wave 34 floats x 64 lanes, lane-contiguous).
    float* const handoff = reinterpret_cast<float*>(smem) + gw * (kHandoffFloats * 64);
    if (group == 1) {
#pragma unroll
        for (int d = 0; d < 2; ++d)
#pragma unroll
            for (int i = 0; i < 16; ++i) handoff[(16 * d + i) * 64 + lane] = o[d][i];
        handoff[32 * 64 + lane] = mc_run;
        handoff[33 * 64 + lane] = l_run;
    }
    __syncthreads();
    if (group == 0) {
        const float mc_other = handoff[32 * 64 + lane];
        const float l_other = handoff[33 * 64 + lane];
        const float mc_new = fmaxf(mc_run, mc_other);
        const float alpha = __builtin_amdgcn_exp2f(mc_run - mc_new);
        const float alpha_other = __builtin_amdgcn_exp2f(mc_other - mc_new);  // 0 when mc_other = -inf
#pragma unroll
        for (int d = 0; d < 2; ++d)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[d][i] = o[d][i] * alpha + handoff[(16 * d + i) * 64 + lane] * alpha_other;
        store_block(o, l_run * alpha + l_other * alpha_other, q_heavy);
    }
}

// Launches through hipModuleLaunchKernel on the kernel's function handle (from
// hipGetFuncBySymbol, cached per device): measured 0.3-0.5 us less host time per
// launch than hipLaunchKernelGGL, and small problems run eagerly are bound by the
// host's launch rate. Every forward kernel takes the same arguments.
using ForwardKernel = void (*)(const _Float16*, const _Float16*, const _Float16*, _Float16*, int, int, float);
constexpr int kMaxDevices = 64;

template <ForwardKernel kKernel>
hipError_t launch_kernel(unsigned grid, unsigned block, hipStream_t stream, const void* q, const void* k,
                         const void* v, void* o, int seq_len, int tiles, float scale_log2) {
    static std::atomic<hipFunction_t> functions[kMaxDevices];
    int device = 0;
    hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess) return err;
    hipFunction_t function = device < kMaxDevices ? functions[device].load(std::memory_order_acquire) : nullptr;
    if (function == nullptr) {
        err = hipGetFuncBySymbol(&function, reinterpret_cast<const void*>(kKernel));
        if (err != hipSuccess) return err;
        if (device < kMaxDevices) functions[device].store(function, std::memory_order_release);
    }
    const _Float16* qh = static_cast<const _Float16*>(q);
    const _Float16* kh = static_cast<const _Float16*>(k);
    const _Float16* vh = static_cast<const _Float16*>(v);
    _Float16* oh = static_cast<_Float16*>(o);
    void* params[] = {&qh, &kh, &vh, &oh, &seq_len, &tiles, &scale_log2};
    return hipModuleLaunchKernel(function, grid, 1, 1, block, 1, 1, 0, stream, params, nullptr);
}

// kPartial instantiations (seq_len not a multiple of the 64-key tile) carry the
// bounds checks of a partial last query block and key tile; the others have none.
template <bool kCausal, int kSplit, int kBlocks>
hipError_t launch_splitk(const void* q, const void* k, const void* v, void* o,
                         int64_t batch_heads, int64_t seq_len, float scale_log2,
                         hipStream_t stream) {
    const int64_t query_blocks = (seq_len + kQueriesPerWave - 1) / kQueriesPerWave;
    const unsigned grid = (unsigned)(batch_heads * query_blocks);
    if (seq_len % (32 * kBlocks) != 0)
        return launch_kernel<fa2_forward_splitk_kernel<kCausal, true, kSplit, kBlocks>>(
            grid, kSplit * 64, stream, q, k, v, o, (int)seq_len, (int)query_blocks, scale_log2);
    return launch_kernel<fa2_forward_splitk_kernel<kCausal, false, kSplit, kBlocks>>(
        grid, kSplit * 64, stream, q, k, v, o, (int)seq_len, (int)query_blocks, scale_log2);
}

template <bool kCausal, int kSplit, int kBlocks>
hipError_t launch_splitk_dma_waves(const void* q, const void* k, const void* v, void* o,
                                   int64_t batch_heads, int64_t seq_len, float scale_log2,
                                   hipStream_t stream) {
    const int64_t query_blocks = (seq_len + kQueriesPerWave - 1) / kQueriesPerWave;
    const unsigned grid = (unsigned)(batch_heads * query_blocks);
    if (seq_len % (32 * kBlocks) != 0)
        return launch_kernel<fa2_forward_splitk_dma_waves_kernel<kCausal, true, kSplit, kBlocks>>(
            grid, 2 * kSplit * 64, stream, q, k, v, o, (int)seq_len, (int)query_blocks, scale_log2);
    return launch_kernel<fa2_forward_splitk_dma_waves_kernel<kCausal, false, kSplit, kBlocks>>(
        grid, 2 * kSplit * 64, stream, q, k, v, o, (int)seq_len, (int)query_blocks, scale_log2);
}

template <int kSplit>
hipError_t launch_pairs16(const void* q, const void* k, const void* v, void* o, int64_t batch_heads,
                          int64_t seq_len, float scale_log2, hipStream_t stream) {
    const int64_t pairs = seq_len / 32;  // 16-query blocks per head, paired
    return launch_kernel<fa2_forward_pairs16_kernel<kSplit>>((unsigned)(batch_heads * pairs), kSplit * 64, stream,
                                                             q, k, v, o, (int)seq_len, (int)pairs, scale_log2);
}

template <bool kCausal, int kWaves>
hipError_t launch_forward(const void* q, const void* k, const void* v, void* o,
                          int64_t batch_heads, int64_t seq_len, float scale_log2,
                          hipStream_t stream) {
    const int64_t block_m = (int64_t)kWaves * kQueriesPerWave;
    const int64_t query_tiles = seq_len / block_m;
    return launch_kernel<fa2_forward_d64_kernel<kCausal, kWaves>>((unsigned)(batch_heads * query_tiles), kWaves * 64,
                                                                  stream, q, k, v, o, (int)seq_len, (int)query_tiles,
                                                                  scale_log2);
}

template <bool kCausal, bool kPairs>
hipError_t launch_wide(const void* q, const void* k, const void* v, void* o, int64_t batch_heads,
                       int64_t seq_len, float scale_log2, hipStream_t stream) {
    const int64_t query_tiles = seq_len / 256;
    const int64_t items = kPairs ? query_tiles / 2 : query_tiles;
    return launch_kernel<fa2_forward_d64_wide_kernel<kCausal, kPairs>>((unsigned)(batch_heads * items), 256, stream, q,
                                                                       k, v, o, (int)seq_len, (int)query_tiles,
                                                                       scale_log2);
}
hipError_t launch_split_pairs(const void* q, const void* k, const void* v, void* o, int64_t batch_heads,
                              int64_t seq_len, float scale_log2, hipStream_t stream) {
    const int64_t query_tiles = seq_len / 128;
    return launch_kernel<fa2_forward_d64_split_pairs_kernel>((unsigned)(batch_heads * (query_tiles / 2)), 512, stream,
                                                             q, k, v, o, (int)seq_len, (int)query_tiles, scale_log2);
}

// Causal 256-query problems with T = 2, 4 or 8 query tiles per head run pairs of tiles
// (T-1-p, then p) per workgroup, which give every workgroup the same work; otherwise (T odd
// or T >= 16) one query tile per workgroup in the level order of xcd_work_item (per-XCD
// head groups), whose workgroups share each head's K/V through one L2 (HBM fetch 1.03-1.09x
// Q+K+V at B16 H16 N4096 against 1.8x for pairs). Measured on MI355X with the pairs' diagonal
// tiles run without barriers (same process, graph replays, head groups -> pairs): -13% at
// T = 4 (B16 H16 N1024), -9% (B32 H16 N1024), -4.5% at T = 8 (B8 H16 N2048); at T = 2 -3.6% to
// -5.5% from 2048 to 8192 tiles (B64 to B512 H16 N512, B64 H64 N512, B128 H32 N512); at T = 16
// and 32 -0.6% to -1.7% (B16 H16 N4096, B8 H32 N4096, B32 H16 N4096, B4 and B8 H16 N8192) and
// -1.1% at T = 64 (B2 H32 N16384), where the groups' lower traffic is kept.
// When batch*heads is not a multiple of 8 the XCD ranges split heads, and an XCD whose
// range holds a split head's heavy tiles gets more work: up to 8/batch_heads of a head's
// share more (5.5% at 36 heads; 82% for one head), so single tiles need 32 heads or more
// there: -28% to -32% at B1 H66 N4096 and B1 H130 N2048 (with the level order).
bool use_head_groups(int64_t batch_heads, int64_t tiles_per_head) {
    if (tiles_per_head % 2 != 0) return true;
    if (batch_heads % 8 != 0 && batch_heads < 32) return false;
    return tiles_per_head >= 16;
}

// 256-query workgroups (64 queries per wave) once the grid fills every workgroup
// slot of the chip (two per CU); below that the 128-query kernel is faster. A
// causal workgroup takes a pair of query tiles when a head has an even number of
// them, so such a problem needs twice the tiles: measured on MI355X, at 512
// workgroups and above the wide kernel runs causal problems 5-12% faster (B16 H16
// N1024, B2 H16 N8192, B1 H64 N4096, B16 H16 N4096) and at 256 it runs them 11-40%
// slower (B1 H32 N4096, B1 H8 N16384). Causal problems with an odd number of tiles
// per head run one tile per workgroup, and only from 2048 workgroups, where that
// schedule was measured no slower than the 128-query kernel.
//
// Noncausal grids that end in a partial round: both kernels run two workgroups per
// CU (512 slots), and a last round of at most 256 workgroups runs them one per CU,
// each faster than when it shares its CU but with the chip half empty. Time model in
// rounds of the wide kernel: `full` rounds of 1, a last round of 1 when more than half
// full, else 0.645 (wide) or 0.58 (128-query: 1.29x and 1.72x a shared workgroup's
// rate alone on a CU, measured with LDS padding); the 128-query kernel's rounds cost
// 0.5375 (half the work, 7.5% slower per FLOP). It runs the grid when its modeled time
// is more than 5% shorter. Measured on MI355X (same process, wide -> 128-query): -15%
// at 576 wide workgroups (B9 H8 N2048, B1 H36 N4096), -13% at 640 (B5 H16 N2048,
// B1 H40 N4096), -4% at 768, +1% at 896, +2.4% at 1280, +7.5% at 1536 and 4096.
double modeled_rounds(int64_t workgroups, double lone_round) {
    const int64_t full = workgroups / 512;
    const int64_t rest = workgroups % 512;
    return (double)full + (rest == 0 ? 0.0 : rest <= 256 ? lone_round : 1.0);
}

bool use_wide_kernel(int64_t batch_heads, int64_t seq_len, bool causal) {
    if (seq_len % 256 != 0) return false;
    const int64_t tiles = seq_len / 256;
    if (causal && tiles % 2 != 0) return batch_heads * tiles >= 2048;
    const int64_t workgroups = batch_heads * (causal ? tiles / 2 : tiles);
    if (workgroups < 512) return false;
    if (causal) return true;
    const double wide = modeled_rounds(workgroups, 0.645);
    const double narrow = 0.5375 * modeled_rounds(2 * workgroups, 0.58);
    return !(narrow < 0.95 * wide);
}

// 128-query workgroups (4 waves) when they fill the chip (two per CU); otherwise
// the key-split kernel (one 32-query block per workgroup, keys split over 4 waves).
// Kernel choice from measured crossovers on MI355X (B*H*N/128 = number of
// 128-query groups): noncausal from 200 groups, causal from 320 groups (fewer
// leave CUs idle behind the longest causal groups). Noncausal, re-measured with the
// routing check (same process, graph replays, key-split 32 -> 128-query): -16% to -28%
// at 200-248 groups (B1 H25-H31 N1024, B2 H13 N1024, B1 H13-H14 N2048, B1 H7 N4096,
// B1 H50-H60 N512), -3% to -7% at 160-192 groups of 1024 keys, +0.5% and +2.3% at 192
// groups of 2048 and 4096 keys. Measured against the key-split
// kernel with the causal tiles in level-ordered chunks (same process): -2% to -23% at
// 320-504 groups (B1 H40 N1024, B1 H24 N2048, B1 H48 N1024, B1 H56 N1024, B1 H63
// N1024; B1 H20 N2048, B1 H10 N4096, B1 H12 N4096, B1 H44 N1024, B1 H52 N1024, B1 H28
// N1536), +5% to +37% at 256-288 groups (B1 H8 N4096, B1 H16 N2048, B4 H8 N1024,
// B1 H32 N1024, B1 H72 N512). Below that the key-split kernel, with 64-key tiles
// while one workgroup per CU covers the grid (256 or fewer 32-query blocks) and
// 32-key tiles (half the LDS, two workgroups per CU) beyond.
bool use_128_query_kernel(int64_t batch_heads, int64_t seq_len, bool causal) {
    const int64_t groups = batch_heads * (seq_len / 128);
    return groups >= (causal ? 320 : 200);
}

// Causal problems of 320 to 512 groups of 128 queries (one round of the 128-query
// kernel) with long key streams: the split pairs (fa2_forward_d64_split_pairs_kernel,
// one workgroup per CU, 160 to 256 of them). Measured on MI355X against the
// 128-query kernel (same process, graph replays): -6% to -10% at 8192 keys (B1 H5-H8),
// -13% to -16% at 16384 (B1 H3-H4, also with sigma = 2 logits), -16% at B1 H2 N32768;
// with its LDS-staged output and early K/V reads, -3% to -10% at 4096 keys (B1 H10-H16,
// B2 H8, B3 H5), -1.5% to +3% at 2048 keys and 6-13% slower at 1024 keys,
// where its steps and fixed costs (Q, the first tiles, the light tile's store, the
// merge) outweigh the balance. Below 320 groups the key-split kernel with 32-key tiles
// was 10-35% faster at 4096-8192 keys (B1 H6-H8 N4096, B1 H3-H4 N8192) and the split
// pairs gained at most 9% at 256 groups of 16384-32768 keys. Each wave running the 128-query kernel's software
// pipeline instead measured 4-30% slower at every length. Beyond 512 groups the
// 128-query kernel's level order balances its rounds, and the split pairs (several
// rounds of one workgroup per CU) ran 20-45% slower (B1 H10-H16 N8192, B1 H5-H8 N16384).
constexpr int64_t kSplitPairsMinKeys = 4096;
bool use_split_pairs_kernel(int64_t batch_heads, int64_t seq_len, bool causal) {
    if (!causal || seq_len % 256 != 0 || seq_len < kSplitPairsMinKeys) return false;
    const int64_t groups = batch_heads * (seq_len / 128);
    return groups >= 320 && groups <= 512;
}

constexpr int64_t kSplitWideMaxBlocks = 256;
constexpr int64_t kEightWaveMinKeys = 2048;
constexpr int64_t kPairs16MinKeys = 512;
constexpr int64_t kDmaWavesMinKeys = 1024;

// The kernel a forward call with these sizes runs (the single place the choice is made).
fa2_forward_kernel choose_kernel(int64_t batch_heads, int64_t seq_len, bool causal) {
    if (use_wide_kernel(batch_heads, seq_len, causal)) {
        const int64_t tiles = seq_len / 256;
        return causal && tiles % 2 == 0 && !use_head_groups(batch_heads, tiles) ? FA2_KERNEL_256_QUERY_PAIRS
                                                                               : FA2_KERNEL_256_QUERY;
    }
    if (use_split_pairs_kernel(batch_heads, seq_len, causal)) return FA2_KERNEL_128_QUERY_SPLIT_PAIRS;
    if (seq_len % kQueryTileAlign == 0 && use_128_query_kernel(batch_heads, seq_len, causal))
        return FA2_KERNEL_128_QUERY;
    const int64_t query_blocks = (seq_len + kQueriesPerWave - 1) / kQueriesPerWave;
    if (batch_heads * query_blocks > kSplitWideMaxBlocks) return FA2_KERNEL_KEY_SPLIT_32;
    // Causal, one workgroup per CU, from 512 to 2047 keys: pairs of 16-query blocks, so
    // every workgroup has the same key tiles instead of the last block having all of
    // them. Measured on MI355X against 32-query blocks: -13% at B1 H8 N896, -7% at
    // B1 H8 N768, -2% at N512 (-6.5% at B1 H8 N1024 and -16% at B1 H4 N1920 before the
    // light block shared the heavy block's key tiles); 3-7% slower at 128-256 keys.
    if (causal && seq_len % 64 == 0 && seq_len >= kPairs16MinKeys && seq_len < kEightWaveMinKeys)
        return FA2_KERNEL_KEY_SPLIT_PAIRS16;
    // One workgroup per CU: from 2048 keys on, 8 waves with two 32-key stages each
    // halve every wave's chain of tiles, measured 2-6% faster noncausal and 6-13%
    // causal (B1 H1-4 N2048-8192); at 1024 keys and below they are no faster.
    if (seq_len >= kEightWaveMinKeys) return FA2_KERNEL_KEY_SPLIT_8_WAVES;
    // Noncausal, from 1024 keys (four or more 64-key tiles per wave): dedicated DMA
    // waves keep two tiles per wave in flight. Measured on MI355X against the plain
    // key-split kernel: -4% to -5% at B1 H8 N1024 and B1 H1 N1024; below 1024 keys
    // (one to three tiles per wave) it was 3-9% slower.
    if (!causal && seq_len >= kDmaWavesMinKeys) return FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES;
    // Otherwise 4 waves with 64-key tiles when each wave gets the same number of them;
    // else 32-key tiles, which split the keys evenly (or less unevenly) and give short
    // causal blocks more waves. Measured on MI355X (same process, graph replays, 64- ->
    // 32-key tiles): noncausal -6% at N128, -7% at N384, -6% at N640, -3% to -5% at N896
    // (B1 H2-H8), 0 at N256, N512, N768; causal -14% at N128, -5% to -8% at N256, -13%
    // at N384.
    if (causal || ((seq_len + kKeysPerTile - 1) / kKeysPerTile) % 4 != 0) return FA2_KERNEL_KEY_SPLIT_32;
    return FA2_KERNEL_KEY_SPLIT_64;
}

bool misaligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) != 0; }

// Whether `kernel` computes these sizes (a sequence length the production entry accepts,
// a multiple of 128): the shapes each kernel's indexing, tile counts and schedules are
// written for, whether or not choose_kernel routes them there. The 256-query kernel
// fetches three 64-key tiles ahead (N a multiple of 256); its pairs take two 256-query
// tiles per workgroup (causal, N a multiple of 512); the split pairs pair 128-query tiles
// and split each pair's keys over two wave groups (causal, N a multiple of 256, from 1024
// keys); the paired 16-query kernel pairs 16-query blocks (causal, N a multiple of 64,
// from 512 keys); the DMA-waves kernel is noncausal. The 128-query and key-split kernels
// take every such length in both modes.
bool kernel_handles(int kernel, int64_t seq_len, bool causal) {
    switch (kernel) {
        case FA2_KERNEL_256_QUERY: return seq_len % 256 == 0;
        case FA2_KERNEL_256_QUERY_PAIRS: return causal && seq_len % 512 == 0;
        case FA2_KERNEL_128_QUERY: return seq_len % 128 == 0;
        case FA2_KERNEL_128_QUERY_SPLIT_PAIRS: return causal && seq_len % 256 == 0 && seq_len >= 1024;
        case FA2_KERNEL_KEY_SPLIT_64:
        case FA2_KERNEL_KEY_SPLIT_32:
        case FA2_KERNEL_KEY_SPLIT_8_WAVES: return true;
        case FA2_KERNEL_KEY_SPLIT_PAIRS16: return causal && seq_len % 64 == 0 && seq_len >= kPairs16MinKeys;
        case FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES: return !causal;
        default: return false;
    }
}


// Shared argument checks and dispatch of the C entry points. `multiple` is the
// divisor seq_len must have; sequence lengths that are multiples of 256 or 128 run
// the 256- or 128-query kernel when the problem fills the chip, everything else the
// key-split kernel (which handles partial query blocks and key tiles).
int forward(const void* query, const void* key, const void* value, void* output, int64_t batch,
            int64_t heads, int64_t seq_len, int64_t head_dim, int64_t multiple, bool causal,
            void* stream, int forced_kernel = FA2_KERNEL_NONE) {
    if (batch < 0 || heads < 0 || seq_len < 0 || head_dim < 0) return FA2_STATUS_NEGATIVE_DIMENSION;
    if (head_dim != kHeadDim) return FA2_STATUS_BAD_HEAD_DIM;
    if (seq_len % multiple != 0) return FA2_STATUS_BAD_SEQUENCE_LENGTH;
    if (batch == 0 || heads == 0 || seq_len == 0) return FA2_STATUS_SUCCESS;
    if (!query || !key || !value || !output) return FA2_STATUS_NULL_POINTER;
    if (misaligned(query) || misaligned(key) || misaligned(value) || misaligned(output))
        return FA2_STATUS_MISALIGNED;
    // Kernel indexing: byte offsets inside one head's slab are 32-bit (buffer
    // loads), the grid is 1-D.
    if (seq_len > kMaxSeqLen || batch > (int64_t)UINT32_MAX / heads)
        return FA2_STATUS_TOO_LARGE;
    const int64_t batch_heads = batch * heads;
    const int64_t query_blocks = (seq_len + kQueriesPerWave - 1) / kQueriesPerWave;
    if (batch_heads > (int64_t)UINT32_MAX / query_blocks) return FA2_STATUS_TOO_LARGE;

    if (forced_kernel != FA2_KERNEL_NONE && !kernel_handles(forced_kernel, seq_len, causal))
        return FA2_STATUS_BAD_KERNEL;

    const float scale = 1.0f / sqrtf((float)kHeadDim);           // reference :3040-3046
    const float scale_log2 = scale * 1.4426950408889634074f;     // fold log2(e) for exp2
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t err;
    switch (forced_kernel != FA2_KERNEL_NONE ? (fa2_forward_kernel)forced_kernel : choose_kernel(batch_heads, seq_len, causal)) {
        case FA2_KERNEL_256_QUERY:
            err = causal ? launch_wide<true, false>(query, key, value, output, batch_heads, seq_len, scale_log2, s)
                         : launch_wide<false, false>(query, key, value, output, batch_heads, seq_len, scale_log2, s);
            break;
        case FA2_KERNEL_256_QUERY_PAIRS:
            err = launch_wide<true, true>(query, key, value, output, batch_heads, seq_len, scale_log2, s);
            break;
        case FA2_KERNEL_128_QUERY:
            err = causal ? launch_forward<true, 4>(query, key, value, output, batch_heads, seq_len, scale_log2, s)
                         : launch_forward<false, 4>(query, key, value, output, batch_heads, seq_len, scale_log2, s);
            break;
        case FA2_KERNEL_128_QUERY_SPLIT_PAIRS:
            err = launch_split_pairs(query, key, value, output, batch_heads, seq_len, scale_log2, s);
            break;
        case FA2_KERNEL_KEY_SPLIT_64:
            err = causal ? launch_splitk<true, 4, 2>(query, key, value, output, batch_heads, seq_len, scale_log2, s)
                         : launch_splitk<false, 4, 2>(query, key, value, output, batch_heads, seq_len, scale_log2, s);
            break;
        case FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES:
            err = launch_splitk_dma_waves<false, 4, 2>(query, key, value, output, batch_heads, seq_len, scale_log2, s);
            break;
        case FA2_KERNEL_KEY_SPLIT_PAIRS16:
            err = launch_pairs16<4>(query, key, value, output, batch_heads, seq_len, scale_log2, s);
            break;
        case FA2_KERNEL_KEY_SPLIT_8_WAVES:
            err = causal ? launch_splitk<true, 8, 1>(query, key, value, output, batch_heads, seq_len, scale_log2, s)
                         : launch_splitk<false, 8, 1>(query, key, value, output, batch_heads, seq_len, scale_log2, s);
            break;
        default:
            err = causal ? launch_splitk<true, 4, 1>(query, key, value, output, batch_heads, seq_len, scale_log2, s)
                         : launch_splitk<false, 4, 1>(query, key, value, output, batch_heads, seq_len, scale_log2, s);
            break;
    }
    return err == hipSuccess ? FA2_STATUS_SUCCESS : FA2_STATUS_HIP_ERROR_BASE + (int)err;
}

}  // namespace

extern "C" int fa2_forward_production_128x128(const void* query, const void* key,
                                              const void* value, void* output, int64_t batch,
                                              int64_t heads, int64_t seq_len, int64_t head_dim,
                                              int causal, void* stream) {
    return forward(query, key, value, output, batch, heads, seq_len, head_dim, kQueryTileAlign,
                   causal != 0, stream);
}

extern "C" int fa2_forward_tensorcore(const void* query, const void* key, const void* value,
                                      void* output, int64_t batch, int64_t heads,
                                      int64_t seq_len, int64_t head_dim, int64_t key_tile,
                                      void* stream) {
    if (key_tile != 16 && key_tile != 32) return FA2_STATUS_BAD_KEY_TILE;
    return forward(query, key, value, output, batch, heads, seq_len, head_dim, key_tile,
                   /*causal=*/false, stream);
}

extern "C" int fa2_forward_with_kernel(int kernel, const void* query, const void* key,
                                       const void* value, void* output, int64_t batch,
                                       int64_t heads, int64_t seq_len, int64_t head_dim,
                                       int causal, void* stream) {
    if (kernel <= FA2_KERNEL_NONE || kernel > FA2_KERNEL_128_QUERY_SPLIT_PAIRS) return FA2_STATUS_BAD_KERNEL;
    return forward(query, key, value, output, batch, heads, seq_len, head_dim, kQueryTileAlign,
                   causal != 0, stream, kernel);
}

extern "C" const char* fa2_status_string(int status) {
    switch (status) {
        case FA2_STATUS_SUCCESS: return "success";
        case FA2_STATUS_NULL_POINTER: return "null tensor pointer";
        case FA2_STATUS_NEGATIVE_DIMENSION: return "negative dimension";
        case FA2_STATUS_BAD_HEAD_DIM: return "head dimension must equal 64";
        case FA2_STATUS_BAD_SEQUENCE_LENGTH: return "sequence length not a multiple of the entry's key tile";
        case FA2_STATUS_MISALIGNED: return "tensor pointer not 16-byte aligned";
        case FA2_STATUS_TOO_LARGE: return "problem too large for the kernel's launch grid";
        case FA2_STATUS_BAD_KEY_TILE: return "key tile must be 16 or 32";
        case FA2_STATUS_BAD_KERNEL: return "kernel does not compute these sizes";
        default: break;
    }
    if (status > FA2_STATUS_HIP_ERROR_BASE)
        return hipGetErrorString(static_cast<hipError_t>(status - FA2_STATUS_HIP_ERROR_BASE));
    return "unknown status";
}

extern "C" int fa2_forward_plan(int64_t batch, int64_t heads, int64_t seq_len, int causal) {
    if (batch <= 0 || heads <= 0 || seq_len <= 0) return FA2_KERNEL_NONE;
    if (seq_len > kMaxSeqLen || batch > (int64_t)UINT32_MAX / heads) return FA2_KERNEL_NONE;
    const int64_t batch_heads = batch * heads;
    const int64_t query_blocks = (seq_len + kQueriesPerWave - 1) / kQueriesPerWave;
    if (batch_heads > (int64_t)UINT32_MAX / query_blocks) return FA2_KERNEL_NONE;
    return choose_kernel(batch_heads, seq_len, causal != 0);
}

extern "C" int fa2_abi_version(void) { return FA2_MI355X_ABI_VERSION; }
