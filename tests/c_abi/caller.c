/*
 * A plain C caller of the C ABI (include/fa2_mi355x.h), built with gcc against the HIP
 * runtime's C API: what a non-Python host (cgo, JNI, a C service) would do.
 *
 * With Q = K = 0 every score is 0, so the softmax is uniform over the visible keys:
 * noncausal O[i] = mean over all keys of V, causal O[i] = mean of V[0..i]. Those are
 * computed on the host in double and compared with the FP16 output (atol 2e-3 + rtol
 * 1e-2). V[j][d] = ((j * 37 + d * 11) % 101) / 50 - 1 is exact in FP16. Also checks
 * argument rejection, the empty problem and fa2_forward_plan, and the causal closed form at
 * a size the split pairs run (B1 H5 N8192). Prints "ok" and exits 0 when every check passes.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "fa2_mi355x.h"

#define B 2
#define H 3
#define N 256
#define D 64

static int failures = 0;

#define CHECK(cond, ...)                        \
    do {                                        \
        if (!(cond)) {                          \
            fprintf(stderr, __VA_ARGS__);       \
            fprintf(stderr, "\n");              \
            ++failures;                         \
        }                                       \
    } while (0)

/* IEEE binary16 <-> float for values the test uses (normal numbers and zero). */
static uint16_t to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int32_t exp = (int32_t)((x >> 23) & 0xff) - 127 + 15;
    uint32_t mant = x & 0x7fffffu;
    if ((x & 0x7fffffffu) == 0) return (uint16_t)sign;
    /* round to nearest even on the 13 dropped bits */
    uint32_t h = sign | ((uint32_t)exp << 10) | (mant >> 13);
    const uint32_t rest = mant & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)h;
}

static float from_half(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1f;
    const uint32_t mant = h & 0x3ffu;
    uint32_t x;
    if (exp == 0 && mant == 0) x = sign;
    else if (exp == 0x1f) x = sign | 0x7f800000u | (mant << 13);
    else if (exp == 0) { /* subnormal */
        float f = ldexpf((float)mant, -24);
        return (h & 0x8000u) ? -f : f;
    } else x = sign | ((exp - 15 + 127) << 23) | (mant << 13);
    float f;
    memcpy(&f, &x, 4);
    return f;
}

static double v_value(int j, int d) { return (double)((j * 37 + d * 11) % 101) / 50.0 - 1.0; }

/* Causal, Q = K = 0, at a size the causal split pairs run (batch*heads*seq_len/128 = 320,
 * seq_len 8192): O[i] is the mean of V[0..i], from prefix sums. Returns 0 on success. */
static int check_causal_prefix_means(int64_t batch, int64_t heads, int64_t seq_len) {
    const size_t elems = (size_t)(batch * heads * seq_len) * D;
    const size_t bytes = elems * sizeof(uint16_t);
    uint16_t* host_zero = calloc(elems, sizeof(uint16_t));
    uint16_t* host_v = malloc(bytes);
    uint16_t* host_o = malloc(bytes);
    double* prefix = malloc(sizeof(double) * D);
    if (!host_zero || !host_v || !host_o || !prefix) return 2;
    for (int64_t bh = 0; bh < batch * heads; ++bh)
        for (int64_t j = 0; j < seq_len; ++j)
            for (int d = 0; d < D; ++d) host_v[((size_t)bh * seq_len + j) * D + d] = to_half((float)v_value((int)j, d));
    void *q, *k, *v, *o;
    if (hipMalloc(&q, bytes) != hipSuccess || hipMalloc(&k, bytes) != hipSuccess ||
        hipMalloc(&v, bytes) != hipSuccess || hipMalloc(&o, bytes) != hipSuccess)
        return 2;
    hipMemcpy(q, host_zero, bytes, hipMemcpyHostToDevice);
    hipMemcpy(k, host_zero, bytes, hipMemcpyHostToDevice);
    hipMemcpy(v, host_v, bytes, hipMemcpyHostToDevice);
    hipMemset(o, 0xff, bytes); /* NaN pattern: every output must be written */
    const int status = fa2_forward_production_128x128(q, k, v, o, batch, heads, seq_len, D, 1, NULL);
    CHECK(status == FA2_STATUS_SUCCESS, "split pairs: status %d (%s)", status, fa2_status_string(status));
    if (hipDeviceSynchronize() != hipSuccess) return 2;
    hipMemcpy(host_o, o, bytes, hipMemcpyDeviceToHost);
    double worst = 0.0;
    for (int64_t bh = 0; bh < batch * heads; ++bh) {
        for (int d = 0; d < D; ++d) prefix[d] = 0.0;
        for (int64_t i = 0; i < seq_len; ++i)
            for (int d = 0; d < D; ++d) {
                prefix[d] += v_value((int)i, d);
                const double mean = prefix[d] / (double)(i + 1);
                const double got = from_half(host_o[((size_t)bh * seq_len + i) * D + d]);
                if (!(fabs(got - mean) - (2e-3 + 1e-2 * fabs(mean)) <= 0.0)) {
                    ++failures;
                    if (failures < 5)
                        fprintf(stderr, "split pairs bh=%lld i=%lld d=%d: got %f want %f\n", (long long)bh,
                                (long long)i, d, got, mean);
                }
                if (fabs(got - mean) > worst) worst = fabs(got - mean);
            }
    }
    printf("split pairs (B%lld H%lld N%lld causal): max abs error %.3e\n", (long long)batch, (long long)heads,
           (long long)seq_len, worst);
    hipFree(q);
    hipFree(k);
    hipFree(v);
    hipFree(o);
    free(host_zero);
    free(host_v);
    free(host_o);
    free(prefix);
    return 0;
}

int main(void) {
    const size_t elems = (size_t)B * H * N * D;
    const size_t bytes = elems * sizeof(uint16_t);
    uint16_t* host_zero = calloc(elems, sizeof(uint16_t));
    uint16_t* host_v = malloc(bytes);
    uint16_t* host_o = malloc(bytes);
    for (int bh = 0; bh < B * H; ++bh)
        for (int j = 0; j < N; ++j)
            for (int d = 0; d < D; ++d) host_v[((size_t)bh * N + j) * D + d] = to_half((float)v_value(j, d));

    void *q, *k, *v, *o;
    if (hipMalloc(&q, bytes) != hipSuccess || hipMalloc(&k, bytes) != hipSuccess ||
        hipMalloc(&v, bytes) != hipSuccess || hipMalloc(&o, bytes) != hipSuccess) {
        fprintf(stderr, "hipMalloc failed\n");
        return 2;
    }
    hipMemcpy(q, host_zero, bytes, hipMemcpyHostToDevice);
    hipMemcpy(k, host_zero, bytes, hipMemcpyHostToDevice);
    hipMemcpy(v, host_v, bytes, hipMemcpyHostToDevice);

    CHECK(fa2_abi_version() == FA2_MI355X_ABI_VERSION, "ABI version %d", fa2_abi_version());

    for (int causal = 0; causal <= 1; ++causal) {
        hipMemset(o, 0xff, bytes); /* NaN pattern: every output must be written */
        const int status = fa2_forward_production_128x128(q, k, v, o, B, H, N, D, causal, NULL);
        CHECK(status == FA2_STATUS_SUCCESS, "causal=%d: status %d (%s)", causal, status, fa2_status_string(status));
        if (hipDeviceSynchronize() != hipSuccess) {
            fprintf(stderr, "kernel failed\n");
            return 2;
        }
        hipMemcpy(host_o, o, bytes, hipMemcpyDeviceToHost);
        double worst = 0.0;
        for (int bh = 0; bh < B * H; ++bh)
            for (int i = 0; i < N; ++i) {
                const int visible = causal ? i + 1 : N;
                for (int d = 0; d < D; ++d) {
                    double mean = 0.0;
                    for (int j = 0; j < visible; ++j) mean += v_value(j, d);
                    mean /= visible;
                    const double got = from_half(host_o[((size_t)bh * N + i) * D + d]);
                    const double excess = fabs(got - mean) - (2e-3 + 1e-2 * fabs(mean));
                    if (!(excess <= 0.0)) {
                        ++failures;
                        if (failures < 5)
                            fprintf(stderr, "causal=%d bh=%d i=%d d=%d: got %f want %f\n", causal, bh, i, d, got, mean);
                    }
                    if (fabs(got - mean) > worst) worst = fabs(got - mean);
                }
            }
        printf("causal=%d: max abs error %.3e\n", causal, worst);
    }

    /* Rejected arguments: nothing is launched. */
    CHECK(fa2_forward_production_128x128(q, k, v, o, B, H, N, 32, 0, NULL) == FA2_STATUS_BAD_HEAD_DIM, "head_dim 32");
    CHECK(fa2_forward_production_128x128(q, k, v, o, B, H, 200, D, 0, NULL) == FA2_STATUS_BAD_SEQUENCE_LENGTH, "N 200");
    CHECK(fa2_forward_production_128x128(NULL, k, v, o, B, H, N, D, 0, NULL) == FA2_STATUS_NULL_POINTER, "null q");
    CHECK(fa2_forward_production_128x128((char*)q + 2, k, v, o, B, H, N, D, 0, NULL) == FA2_STATUS_MISALIGNED, "misaligned q");
    CHECK(fa2_forward_production_128x128(NULL, NULL, NULL, NULL, 0, H, N, D, 1, NULL) == FA2_STATUS_SUCCESS, "empty batch");
    CHECK(fa2_forward_tensorcore(q, k, v, o, B, H, N, D, 8, NULL) == FA2_STATUS_BAD_KEY_TILE, "key tile 8");
    CHECK(fa2_forward_plan(B, H, N, 0) == FA2_KERNEL_KEY_SPLIT_64, "plan %d", fa2_forward_plan(B, H, N, 0));
    CHECK(fa2_forward_plan(16, 16, 4096, 1) == FA2_KERNEL_256_QUERY, "plan big causal");
    CHECK(fa2_forward_plan(16, 16, 1024, 1) == FA2_KERNEL_256_QUERY_PAIRS, "plan causal pairs");
    CHECK(strcmp(fa2_status_string(FA2_STATUS_BAD_HEAD_DIM), "head dimension must equal 64") == 0, "status text");

    CHECK(fa2_forward_plan(1, 5, 8192, 1) == FA2_KERNEL_128_QUERY_SPLIT_PAIRS, "plan split pairs");
    if (check_causal_prefix_means(1, 5, 8192) != 0) {
        fprintf(stderr, "split pairs check could not run\n");
        return 2;
    }

    hipFree(q);
    hipFree(k);
    hipFree(v);
    hipFree(o);
    free(host_zero);
    free(host_v);
    free(host_o);
    if (failures) {
        fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    printf("ok\n");
    return 0;
}
