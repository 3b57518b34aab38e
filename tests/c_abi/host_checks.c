/*
 * Host-side paths of the C ABI (include/fa2_mi355x.h) that need no GPU: argument
 * rejection and empty problems of every entry point, status strings and the kernel
 * plan. Nothing here launches a kernel or calls the HIP runtime, so it runs on a
 * machine without a GPU. The CPU test suite builds it with AddressSanitizer and
 * UndefinedBehaviorSanitizer against a host-only sanitizer build of the library.
 * Prints "ok" and exits 0 when every check passes.
 */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "fa2_mi355x.h"

static int failures = 0;

#define CHECK(cond, ...)                        \
    do {                                        \
        if (!(cond)) {                          \
            fprintf(stderr, __VA_ARGS__);       \
            fprintf(stderr, "\n");              \
            ++failures;                         \
        }                                       \
    } while (0)

/* Never dereferenced: every call below is rejected (or empty) before any launch. */
static _Alignas(16) unsigned char fake[4][64];

static int forward(const void* q, const void* k, const void* v, void* o, int64_t batch, int64_t heads,
                   int64_t seq_len, int64_t head_dim, int causal) {
    return fa2_forward_production_128x128(q, k, v, o, batch, heads, seq_len, head_dim, causal, NULL);
}

static int tensorcore(const void* q, int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                      int64_t key_tile) {
    return fa2_forward_tensorcore(q, fake[1], fake[2], fake[3], batch, heads, seq_len, head_dim, key_tile, NULL);
}

int main(void) {
    const void *q = fake[0], *k = fake[1], *v = fake[2];
    void* o = fake[3];

    CHECK(fa2_abi_version() == FA2_MI355X_ABI_VERSION, "ABI version %d", fa2_abi_version());

    for (int causal = 0; causal <= 1; ++causal) {
        /* Status precedence: negative sizes, head dim, sequence length, empty, null, alignment, size. */
        CHECK(forward(q, k, v, o, -1, 1, 128, 64, causal) == FA2_STATUS_NEGATIVE_DIMENSION, "negative batch");
        CHECK(forward(q, k, v, o, 1, -1, 128, 64, causal) == FA2_STATUS_NEGATIVE_DIMENSION, "negative heads");
        CHECK(forward(q, k, v, o, 1, 1, -128, 64, causal) == FA2_STATUS_NEGATIVE_DIMENSION, "negative seq_len");
        CHECK(forward(q, k, v, o, 1, 1, 128, -64, causal) == FA2_STATUS_NEGATIVE_DIMENSION, "negative head_dim");
        CHECK(forward(q, k, v, o, 1, 1, 128, 32, causal) == FA2_STATUS_BAD_HEAD_DIM, "head_dim 32");
        CHECK(forward(q, k, v, o, 1, 1, 128, 128, causal) == FA2_STATUS_BAD_HEAD_DIM, "head_dim 128");
        CHECK(forward(NULL, NULL, NULL, NULL, 0, 1, 128, 32, causal) == FA2_STATUS_BAD_HEAD_DIM,
              "empty problem still checks head_dim");
        for (int64_t n = 1; n < 128; n += 17)
            CHECK(forward(q, k, v, o, 1, 1, n, 64, causal) == FA2_STATUS_BAD_SEQUENCE_LENGTH, "seq_len %lld",
                  (long long)n);
        CHECK(forward(q, k, v, o, 1, 1, 200, 64, causal) == FA2_STATUS_BAD_SEQUENCE_LENGTH, "seq_len 200");
        CHECK(forward(NULL, NULL, NULL, NULL, 0, 8, 1024, 64, causal) == FA2_STATUS_SUCCESS, "empty batch");
        CHECK(forward(NULL, NULL, NULL, NULL, 2, 0, 1024, 64, causal) == FA2_STATUS_SUCCESS, "empty heads");
        CHECK(forward(NULL, NULL, NULL, NULL, 2, 8, 0, 64, causal) == FA2_STATUS_SUCCESS, "empty sequence");
        CHECK(forward(NULL, k, v, o, 1, 1, 128, 64, causal) == FA2_STATUS_NULL_POINTER, "null query");
        CHECK(forward(q, NULL, v, o, 1, 1, 128, 64, causal) == FA2_STATUS_NULL_POINTER, "null key");
        CHECK(forward(q, k, NULL, o, 1, 1, 128, 64, causal) == FA2_STATUS_NULL_POINTER, "null value");
        CHECK(forward(q, k, v, NULL, 1, 1, 128, 64, causal) == FA2_STATUS_NULL_POINTER, "null output");
        for (int shift = 1; shift < 16; ++shift) {
            const unsigned char* bad = fake[0] + shift;
            CHECK(forward(bad, k, v, o, 1, 1, 128, 64, causal) == FA2_STATUS_MISALIGNED, "query + %d", shift);
            CHECK(forward(q, bad, v, o, 1, 1, 128, 64, causal) == FA2_STATUS_MISALIGNED, "key + %d", shift);
            CHECK(forward(q, k, bad, o, 1, 1, 128, 64, causal) == FA2_STATUS_MISALIGNED, "value + %d", shift);
            CHECK(forward(q, k, v, (void*)bad, 1, 1, 128, 64, causal) == FA2_STATUS_MISALIGNED, "output + %d", shift);
        }
        /* Beyond the 32-bit slab offsets and the 1-D grid; products near INT64_MAX must not overflow. */
        CHECK(forward(q, k, v, o, 1, 1, ((int64_t)1 << 24) + 128, 64, causal) == FA2_STATUS_TOO_LARGE, "seq_len 2^24+128");
        CHECK(forward(q, k, v, o, (int64_t)1 << 40, (int64_t)1 << 40, 128, 64, causal) == FA2_STATUS_TOO_LARGE,
              "batch * heads beyond int64");
        CHECK(forward(q, k, v, o, INT64_MAX, 1, 128, 64, causal) == FA2_STATUS_TOO_LARGE, "batch INT64_MAX");
        CHECK(forward(q, k, v, o, 1, INT64_MAX, 128, 64, causal) == FA2_STATUS_TOO_LARGE, "heads INT64_MAX");
        CHECK(forward(q, k, v, o, (int64_t)1 << 31, 1 << 12, 1 << 12, 64, causal) == FA2_STATUS_TOO_LARGE,
              "grid beyond 2^32 groups");
        CHECK(forward(q, k, v, o, INT64_MAX, INT64_MAX, INT64_MAX, 64, causal) == FA2_STATUS_BAD_SEQUENCE_LENGTH,
              "INT64_MAX sizes");
    }

    /* fa2_forward_tensorcore: key tile 16 or 32, seq_len a multiple of it, same other checks.
     * The key tile is checked first; a null query stops an accepted tile before any launch. */
    for (int64_t tile = -1; tile <= 64; ++tile) {
        const int status = tensorcore(NULL, 1, 1, 64, 64, tile);
        if (tile == 16 || tile == 32)
            CHECK(status == FA2_STATUS_NULL_POINTER, "key tile %lld: status %d", (long long)tile, status);
        else
            CHECK(status == FA2_STATUS_BAD_KEY_TILE, "key tile %lld: status %d", (long long)tile, status);
    }
    CHECK(tensorcore(q, 1, 1, 48, 64, 32) == FA2_STATUS_BAD_SEQUENCE_LENGTH, "48 keys, tile 32");
    CHECK(tensorcore(q, 1, 1, 40, 64, 16) == FA2_STATUS_BAD_SEQUENCE_LENGTH, "40 keys, tile 16");
    CHECK(tensorcore(q, 1, 1, 48, 32, 16) == FA2_STATUS_BAD_HEAD_DIM, "tensorcore head_dim");
    CHECK(tensorcore(NULL, 1, 1, 48, 64, 16) == FA2_STATUS_NULL_POINTER, "tensorcore null query");
    CHECK(tensorcore(fake[0] + 8, 1, 1, 48, 64, 16) == FA2_STATUS_MISALIGNED, "tensorcore misaligned query");
    CHECK(tensorcore(NULL, 0, 1, 48, 64, 16) == FA2_STATUS_SUCCESS, "tensorcore empty batch");

    /* fa2_forward_with_kernel: an unknown kernel id is rejected first; a known one goes through
     * the production checks (a null query stops it before any launch), then its domain. Only
     * sizes outside the chosen kernel's domain get past the pointer checks here. */
    for (int kernel = -2; kernel <= 12; ++kernel)
        for (int causal = 0; causal <= 1; ++causal) {
            const int known = kernel >= FA2_KERNEL_256_QUERY && kernel <= FA2_KERNEL_128_QUERY_SPLIT_PAIRS;
            const int status = fa2_forward_with_kernel(kernel, NULL, k, v, o, 1, 1, 1024, 64, causal, NULL);
            CHECK(status == (known ? FA2_STATUS_NULL_POINTER : FA2_STATUS_BAD_KERNEL), "kernel %d: status %d",
                  kernel, status);
        }
    const int64_t lengths[] = {128, 256, 384, 512, 640, 768, 896, 1024, 1152, 1280, 2048, 4096};
    for (size_t i = 0; i < sizeof(lengths) / sizeof(lengths[0]); ++i)
        for (int causal = 0; causal <= 1; ++causal) {
            const int64_t n = lengths[i];
            const int outside[] = {
                n % 256 != 0 ? FA2_KERNEL_256_QUERY : 0,
                !causal || n % 512 != 0 ? FA2_KERNEL_256_QUERY_PAIRS : 0,
                !causal || n % 256 != 0 || n < 1024 ? FA2_KERNEL_128_QUERY_SPLIT_PAIRS : 0,
                !causal || n % 64 != 0 || n < 512 ? FA2_KERNEL_KEY_SPLIT_PAIRS16 : 0,
                causal ? FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES : 0};
            for (size_t j = 0; j < sizeof(outside) / sizeof(outside[0]); ++j)
                if (outside[j])
                    CHECK(fa2_forward_with_kernel(outside[j], q, k, v, o, 1, 1, n, 64, causal, NULL) ==
                              FA2_STATUS_BAD_KERNEL,
                          "kernel %d outside its domain at %lld keys causal=%d", outside[j], (long long)n, causal);
        }
    CHECK(fa2_forward_with_kernel(FA2_KERNEL_256_QUERY, q, k, v, o, 1, 1, 100, 64, 0, NULL) ==
              FA2_STATUS_BAD_SEQUENCE_LENGTH, "forced kernel, seq_len 100");
    CHECK(fa2_forward_with_kernel(FA2_KERNEL_256_QUERY, q, k, v, o, INT64_MAX, INT64_MAX, 256, 64, 0, NULL) ==
              FA2_STATUS_TOO_LARGE, "forced kernel, sizes beyond the grid");

    /* Every status has a text; unknown codes have one too (static storage, never NULL). */
    const int codes[] = {FA2_STATUS_SUCCESS, FA2_STATUS_NULL_POINTER, FA2_STATUS_NEGATIVE_DIMENSION,
                         FA2_STATUS_BAD_HEAD_DIM, FA2_STATUS_BAD_SEQUENCE_LENGTH, FA2_STATUS_MISALIGNED,
                         FA2_STATUS_TOO_LARGE, FA2_STATUS_BAD_KEY_TILE, FA2_STATUS_BAD_KERNEL,
                         FA2_STATUS_HIP_ERROR_BASE + 1, FA2_STATUS_HIP_ERROR_BASE + 98, -1, 9, 999,
                         INT32_MAX, INT32_MIN};
    for (size_t i = 0; i < sizeof(codes) / sizeof(codes[0]); ++i) {
        const char* text = fa2_status_string(codes[i]);
        CHECK(text != NULL && strlen(text) > 0, "status %d has no text", codes[i]);
    }
    CHECK(strcmp(fa2_status_string(FA2_STATUS_BAD_HEAD_DIM), "head dimension must equal 64") == 0, "head dim text");

    /* The plan is a pure function of the sizes, defined for every input: NONE for empty or
     * negative sizes, seq_len > 2^24 and grids beyond 2^32 32-query blocks; a kernel
     * otherwise (the plan does not check the entry's seq_len multiple). */
    const int64_t sizes[] = {-1, 0, 1, 16, 17, 32, 48, 64, 96, 128, 200, 256, 384, 512, 768, 1024, 1040,
                             2048, 4096, 8192, 16384, (int64_t)1 << 24, ((int64_t)1 << 24) + 256, INT64_MAX};
    const int64_t counts[] = {-1, 0, 1, 2, 3, 8, 16, 32, 64, 256, 4096, (int64_t)1 << 31, INT64_MAX};
    const size_t ns = sizeof(sizes) / sizeof(sizes[0]), nc = sizeof(counts) / sizeof(counts[0]);
    for (size_t a = 0; a < nc; ++a)
        for (size_t b = 0; b < nc; ++b)
            for (size_t c = 0; c < ns; ++c)
                for (int causal = 0; causal <= 1; ++causal) {
                    const int64_t batch = counts[a], heads = counts[b], n = sizes[c];
                    const int plan = fa2_forward_plan(batch, heads, n, causal);
                    CHECK(plan >= FA2_KERNEL_NONE && plan <= FA2_KERNEL_128_QUERY_SPLIT_PAIRS, "plan %d", plan);
                    int none = batch <= 0 || heads <= 0 || n <= 0 || n > ((int64_t)1 << 24);
                    if (!none) none = batch > (int64_t)UINT32_MAX / heads;
                    if (!none) none = batch * heads > (int64_t)UINT32_MAX / ((n + 31) / 32);
                    CHECK((plan == FA2_KERNEL_NONE) == none, "plan %d for %lld %lld %lld causal=%d", plan,
                          (long long)batch, (long long)heads, (long long)n, causal);
                }
    /* The module's other entry points: rejected and empty calls only (valid sizes would launch). */
    const float* fq = (const float*)fake[0];
    float* fo = (float*)fake[3];
    CHECK(fa2_copy(fake[0], fake[1], -1, NULL) == FA2_STATUS_NEGATIVE_DIMENSION, "copy negative");
    CHECK(fa2_copy(NULL, NULL, 0, NULL) == FA2_STATUS_SUCCESS, "copy empty");
    CHECK(fa2_copy(NULL, fake[1], 16, NULL) == FA2_STATUS_NULL_POINTER, "copy null source");
    CHECK(fa2_copy(fake[0], NULL, 16, NULL) == FA2_STATUS_NULL_POINTER, "copy null destination");
    {
        /* Lengths beyond int32 and counts beyond the 2^32-workgroup grid: rejected whatever
         * the other sizes (a count that fits the grid would launch). */
        const int64_t long_len[] = {(int64_t)INT32_MAX + 1, INT64_MAX - 1, INT64_MAX};
        const int64_t big_count[] = {(int64_t)UINT32_MAX + 1, INT64_MAX - 1, INT64_MAX};
        for (size_t i = 0; i < 3; ++i) {
            CHECK(fa2_attention_scores_f32(fq, fq, fo, 1, long_len[i], 64, NULL) == FA2_STATUS_TOO_LARGE,
                  "scores seq_len %lld", (long long)long_len[i]);
            CHECK(fa2_attention_scores_f32(fq, fq, fo, 1, 64, long_len[i], NULL) == FA2_STATUS_TOO_LARGE,
                  "scores head_dim %lld", (long long)long_len[i]);
            CHECK(fa2_attention_scores_f32(fq, fq, fo, big_count[i], 64, 64, NULL) == FA2_STATUS_TOO_LARGE,
                  "scores batch_heads %lld", (long long)big_count[i]);
            CHECK(fa2_attention_forward_f32(fq, fq, fq, fo, 1, long_len[i], 64, NULL) == FA2_STATUS_TOO_LARGE,
                  "f32 forward seq_len %lld", (long long)long_len[i]);
            CHECK(fa2_attention_forward_f32(fq, fq, fq, fo, big_count[i], 64, 128, NULL) == FA2_STATUS_TOO_LARGE,
                  "f32 forward batch_heads %lld", (long long)big_count[i]);
            CHECK(fa2_matmul_16x64x16_f16(fake[0], fake[1], fo, big_count[i], NULL) == FA2_STATUS_TOO_LARGE,
                  "matmul batch %lld", (long long)big_count[i]);
        }
    }
    CHECK(fa2_attention_scores_f32(fq, fq, fo, -1, 64, 64, NULL) == FA2_STATUS_NEGATIVE_DIMENSION, "scores negative");
    CHECK(fa2_attention_scores_f32(NULL, NULL, NULL, 0, 64, 64, NULL) == FA2_STATUS_SUCCESS, "scores empty");
    CHECK(fa2_attention_scores_f32(NULL, fq, fo, 1, 64, 64, NULL) == FA2_STATUS_NULL_POINTER, "scores null");
    CHECK(fa2_attention_scores_f32((const float*)(fake[0] + 2), fq, fo, 1, 64, 64, NULL) == FA2_STATUS_MISALIGNED,
          "scores misaligned");
    CHECK(fa2_attention_forward_f32(fq, fq, fq, fo, 1, 64, 96, NULL) == FA2_STATUS_BAD_HEAD_DIM, "f32 head_dim 96");
    CHECK(fa2_attention_forward_f32(fq, fq, fq, fo, 1, -1, 64, NULL) == FA2_STATUS_NEGATIVE_DIMENSION, "f32 negative");
    CHECK(fa2_attention_forward_f32(NULL, NULL, NULL, NULL, 1, 0, 64, NULL) == FA2_STATUS_SUCCESS, "f32 empty");
    CHECK(fa2_attention_forward_f32(fq, fq, NULL, fo, 1, 64, 64, NULL) == FA2_STATUS_NULL_POINTER, "f32 null value");
    CHECK(fa2_matmul_16x64x16_f16(fake[0], fake[1], fo, -1, NULL) == FA2_STATUS_NEGATIVE_DIMENSION, "matmul negative");
    CHECK(fa2_matmul_16x64x16_f16(NULL, NULL, NULL, 0, NULL) == FA2_STATUS_SUCCESS, "matmul empty");
    CHECK(fa2_matmul_16x64x16_f16(fake[0], NULL, fo, 1, NULL) == FA2_STATUS_NULL_POINTER, "matmul null");
    CHECK(fa2_matmul_16x64x16_f16(fake[0] + 1, fake[1], fo, 1, NULL) == FA2_STATUS_MISALIGNED, "matmul misaligned");

    CHECK(fa2_forward_plan(1, 8, 1024, 0) == FA2_KERNEL_KEY_SPLIT_64_DMA_WAVES, "plan bench size");
    CHECK(fa2_forward_plan(1, 8, 768, 0) == FA2_KERNEL_KEY_SPLIT_64, "plan below 1024 keys");
    CHECK(fa2_forward_plan(1, 8, 896, 0) == FA2_KERNEL_KEY_SPLIT_32, "plan with an uneven 64-key split");
    CHECK(fa2_forward_plan(16, 16, 4096, 0) == FA2_KERNEL_256_QUERY, "plan throughput size");
    CHECK(fa2_forward_plan(16, 16, 4096, 1) == FA2_KERNEL_256_QUERY, "plan throughput size causal");
    CHECK(fa2_forward_plan(16, 16, 1024, 1) == FA2_KERNEL_256_QUERY_PAIRS, "plan causal pairs");
    CHECK(fa2_forward_plan(1, 8, 8192, 1) == FA2_KERNEL_128_QUERY_SPLIT_PAIRS, "plan split pairs");
    CHECK(fa2_forward_plan(1, 9, 8192, 1) == FA2_KERNEL_128_QUERY, "plan beyond one round of split pairs");

    if (failures) {
        fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    printf("ok\n");
    return 0;
}
