/*
 * sanity_main.c -- drives every function of the CPU oracle under AddressSanitizer and
 * UndefinedBehaviorSanitizer (host only; `make -C oracle sanitize` builds lib/oracle_sanity).
 *
 * TEST INFRASTRUCTURE ONLY, like the oracle itself. Every buffer is allocated at exactly the
 * size the function's contract names, so a read or write one element past it is reported.
 * Shapes cover the edges the reference's tests use: single rows and columns, ragged counts
 * (M not a multiple of the thread count, N not a multiple of 16), K = 4 / 32 / 64 minimum
 * blocks, padding wider than the kernel, strides and dilations, and inputs holding NaN, +-inf,
 * subnormals and zeros. Beyond the sanitizers it checks the identities that need no second
 * implementation: threaded forms == single-threaded, sparse GEMM == dense GEMM of the
 * decompressed weights, unpack(pack(meta)) == meta, gemm_dequant == gemm_s32 + epilogue.
 * Exit status 0 when every check holds.
 */
#include "forge_oracle.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static int g_fail = 0;
#define CHECK(cond, ...)                                             \
    do {                                                             \
        if (!(cond)) {                                               \
            fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__);     \
            fprintf(stderr, __VA_ARGS__);                            \
            fprintf(stderr, "\n");                                   \
            g_fail = 1;                                              \
        }                                                            \
    } while (0)

static uint32_t g_rng = 12345u;
static uint32_t rnd(void) {
    g_rng = g_rng * 1664525u + 1013904223u;
    return g_rng >> 8;
}

static void* xmalloc(size_t n) {
    void* p = malloc(n ? n : 1);
    if (!p) {
        fprintf(stderr, "out of memory\n");
        exit(2);
    }
    return p;
}

/* fp16 values: mostly ordinary magnitudes, some specials (NaN, +-inf, subnormals, zeros). */
static void fill_f16(uint16_t* x, size_t n, int specials) {
    static const uint16_t sp[] = {0x7E00, 0xFC00, 0x7C00, 0x0001, 0x8003, 0x0000, 0x8000, 0x7BFF, 0x3C00};
    for (size_t i = 0; i < n; i++) {
        const uint32_t r = rnd();
        if (specials && r % 37 == 0) x[i] = sp[(r >> 6) % (sizeof sp / sizeof sp[0])];
        else x[i] = orc_f32_to_f16(((float)(r % 20001) - 10000.0f) / 4000.0f);
    }
}
static void fill_i8(int8_t* x, size_t n) {
    for (size_t i = 0; i < n; i++) x[i] = (int8_t)((int)(rnd() % 255) - 127);
}
static void fill_scales(uint16_t* s, int n) {
    for (int i = 0; i < n; i++) s[i] = orc_f32_to_f16(0.001f + (float)(rnd() % 1000) / 20000.0f);
}

static void check_conversions(void) {
    for (uint32_t h = 0; h < 65536; h++) {
        const float f = orc_f16_to_f32((uint16_t)h);
        if (f == f) CHECK(orc_f32_to_f16(f) == (uint16_t)h, "f16 round trip %04x", h);
    }
}

static void check_linear(int M, int K, int N, int specials) {
    uint16_t* x = xmalloc((size_t)M * K * 2);
    int8_t* q = xmalloc((size_t)M * K);
    float* s = xmalloc((size_t)M * 4);
    int8_t* W = xmalloc((size_t)N * K);
    uint16_t* ws = xmalloc((size_t)N * 2);
    uint16_t* b = xmalloc((size_t)N * 2);
    int32_t* acc = xmalloc((size_t)M * N * 4);
    int32_t* acc_mt = xmalloc((size_t)M * N * 4);
    uint16_t* y = xmalloc((size_t)M * N * 2);
    uint16_t* y2 = xmalloc((size_t)M * N * 2);
    uint16_t* y3 = xmalloc((size_t)M * N * 2);
    float* wsum = xmalloc((size_t)M * N * 4);
    fill_f16(x, (size_t)M * K, specials);
    fill_i8(W, (size_t)N * K);
    fill_scales(ws, N);
    fill_f16(b, N, 0);

    orc_quantize_rows(x, q, s, M, K);
    orc_gemm_s32(q, W, acc, M, K, N);
    orc_gemm_s32_mt(q, W, acc_mt, M, K, N, 3);
    CHECK(memcmp(acc, acc_mt, (size_t)M * N * 4) == 0, "gemm_s32_mt M=%d K=%d N=%d", M, K, N);
    orc_gemm_s32_rows(q, W, acc_mt, 0, M, K, N);
    CHECK(memcmp(acc, acc_mt, (size_t)M * N * 4) == 0, "gemm_s32_rows");

    orc_dequant_epilogue(acc, s, ws, b, y, M, N);
    orc_gemm_dequant(q, W, s, ws, b, y2, M, K, N);
    CHECK(memcmp(y, y2, (size_t)M * N * 2) == 0, "gemm_dequant vs epilogue M=%d K=%d N=%d", M, K, N);
    orc_gemm_dequant_mt(q, W, s, ws, b, y3, M, K, N, 5);
    CHECK(memcmp(y, y3, (size_t)M * N * 2) == 0, "gemm_dequant_mt");
    orc_linear(x, W, ws, b, y3, M, K, N);
    CHECK(memcmp(y, y3, (size_t)M * N * 2) == 0, "linear");
    orc_gemm_dequant(q, W, s, ws, NULL, y2, M, K, N);
    orc_dequantize_bias(acc, s, ws, NULL, y3, M, N);
    orc_dequantize_bias(acc, s, ws, b, y3, M, N);

    for (size_t i = 0; i < (size_t)M * N; i++) wsum[i] = (float)acc[i] * 0.001f;
    orc_splitk_reduce(wsum, b, y2, M, N);
    orc_splitk_reduce(wsum, NULL, y2, M, N);
    (void)orc_time_gemm_dequant_rows(q, W, s, ws, b, y2, M, K, N);
    (void)orc_time_gemm_dequant_rows_mt(q, W, s, ws, b, y2, M, K, N, 4);

    free(x); free(q); free(s); free(W); free(ws); free(b); free(acc); free(acc_mt);
    free(y); free(y2); free(y3); free(wsum);
}

static void check_sparse(int M, int K, int N) {
    int8_t* w = xmalloc((size_t)N * K);
    int8_t* comp = xmalloc((size_t)N * K / 2);
    uint8_t* meta = xmalloc((size_t)N * K / 4);
    uint8_t* meta2 = xmalloc((size_t)N * K / 4);
    uint32_t* pref = xmalloc((size_t)N * K / 32 * 4);
    uint32_t* pg = xmalloc((size_t)N * K / 32 * 4);
    int8_t* wd = xmalloc((size_t)N * K);
    int8_t* x = xmalloc((size_t)M * K);
    int32_t* c1 = xmalloc((size_t)M * N * 4);
    int32_t* c2 = xmalloc((size_t)M * N * 4);
    int32_t* c3 = xmalloc((size_t)M * N * 4);
    fill_i8(w, (size_t)N * K);
    for (size_t i = 0; i < (size_t)N * K; i += 7) w[i] = 0;   /* ties and zero groups */
    fill_i8(x, (size_t)M * K);
    orc_prune_compress_24(w, comp, meta, N, K);
    orc_decompress_24(comp, meta, wd, N, K);
    orc_pack_metadata_ref(meta, pref, N, K);
    orc_pack_metadata_gfx950(meta, pg, N, K);
    orc_unpack_metadata_gfx950(pg, meta2, N, K);
    CHECK(memcmp(meta, meta2, (size_t)N * K / 4) == 0, "unpack(pack) N=%d K=%d", N, K);
    orc_sparse_gemm_s32(comp, x, meta, c1, M, K, N);
    orc_sparse_gemm_s32_mt(comp, x, meta, c2, M, K, N, 3);
    orc_gemm_s32(x, wd, c3, M, K, N);
    CHECK(memcmp(c1, c2, (size_t)M * N * 4) == 0, "sparse_mt M=%d K=%d N=%d", M, K, N);
    CHECK(memcmp(c1, c3, (size_t)M * N * 4) == 0, "sparse vs dense of decompressed M=%d K=%d N=%d", M, K, N);
    free(w); free(comp); free(meta); free(meta2); free(pref); free(pg); free(wd); free(x);
    free(c1); free(c2); free(c3);
}

static void check_weight_rows(int N, int K) {
    float* w = xmalloc((size_t)N * K * 4);
    int8_t* q = xmalloc((size_t)N * K);
    uint16_t* s16 = xmalloc((size_t)N * 2);
    float* s32 = xmalloc((size_t)N * 4);
    for (size_t i = 0; i < (size_t)N * K; i++) w[i] = ((float)(rnd() % 2001) - 1000.0f) / 300.0f;
    for (int k = 0; k < K; k++) w[k] = 0.0f;   /* an all-zero row */
    orc_quantize_weight_rows(w, q, s16, s32, N, K);
    free(w); free(q); free(s16); free(s32);
}

static void check_conv(int N, int H, int W, int C, int Co, int k, int pad, int stride, int dil) {
    const int Ho = orc_conv_out_size(H, pad, dil, k, stride), Wo = orc_conv_out_size(W, pad, dil, k, stride);
    if (Ho <= 0 || Wo <= 0) return;
    int8_t* x = xmalloc((size_t)N * H * W * C);
    int8_t* w = xmalloc((size_t)Co * k * k * C);
    int32_t* o1 = xmalloc((size_t)N * Ho * Wo * Co * 4);
    int32_t* o2 = xmalloc((size_t)N * Ho * Wo * Co * 4);
    fill_i8(x, (size_t)N * H * W * C);
    fill_i8(w, (size_t)Co * k * k * C);
    orc_conv2d_nhwc_s32(x, w, o1, N, H, W, C, Co, k, k, pad, pad, stride, stride, dil, dil);
    orc_conv2d_nhwc_s32_mt(x, w, o2, N, H, W, C, Co, k, k, pad, pad, stride, stride, dil, dil, 3);
    CHECK(memcmp(o1, o2, (size_t)N * Ho * Wo * Co * 4) == 0, "conv_mt H=%d W=%d k=%d s=%d d=%d", H, W, k, stride, dil);
    free(x); free(w); free(o1); free(o2);
}

static void check_depthwise(int N, int C, int H, int W, int k, int pad, int stride, int dil, int bias) {
    const int Ho = orc_conv_out_size(H, pad, dil, k, stride), Wo = orc_conv_out_size(W, pad, dil, k, stride);
    if (Ho <= 0 || Wo <= 0) return;
    uint16_t* in = xmalloc((size_t)N * C * H * W * 2);
    int8_t* w = xmalloc((size_t)C * k * k);
    uint16_t* ws = xmalloc((size_t)C * 2);
    uint16_t* b = xmalloc((size_t)C * 2);
    uint16_t* out = xmalloc((size_t)N * C * Ho * Wo * 2);
    fill_f16(in, (size_t)N * C * H * W, 1);
    fill_i8(w, (size_t)C * k * k);
    fill_scales(ws, C);
    fill_f16(b, C, 0);
    orc_depthwise_conv2d(in, w, ws, bias ? b : NULL, out, N, C, H, W, k, k, pad, pad, stride, stride, dil, dil);
    free(in); free(w); free(ws); free(b); free(out);
}

static void check_convt(int N, int C_in, int H, int W, int C_out, int bias) {
    uint16_t* in = xmalloc((size_t)N * C_in * H * W * 2);
    int8_t* w = xmalloc((size_t)4 * C_out * C_in);
    uint16_t* ws = xmalloc((size_t)C_out * 2);
    uint16_t* b = xmalloc((size_t)C_out * 2);
    uint16_t* out = xmalloc((size_t)N * C_out * 4 * H * W * 2);
    int32_t* acc = xmalloc((size_t)N * C_out * 4 * H * W * 4);
    fill_f16(in, (size_t)N * C_in * H * W, 1);
    fill_i8(w, (size_t)4 * C_out * C_in);
    fill_scales(ws, C_out);
    fill_f16(b, C_out, 0);
    orc_conv_transpose2d_k2s2(in, w, ws, bias ? b : NULL, out, acc, N, C_in, H, W, C_out);
    orc_conv_transpose2d_k2s2(in, w, ws, bias ? b : NULL, out, NULL, N, C_in, H, W, C_out);
    orc_conv_transpose2d_k2s2(in, w, ws, bias ? b : NULL, NULL, acc, N, C_in, H, W, C_out);
    free(in); free(w); free(ws); free(b); free(out); free(acc);
}

int main(void) {
    check_conversions();

    static const int lin[][3] = {{1, 1, 1}, {1, 4096, 3}, {7, 33, 17}, {16, 128, 64}, {5, 1, 9}, {64, 96, 48}};
    for (size_t i = 0; i < sizeof lin / sizeof lin[0]; i++) {
        check_linear(lin[i][0], lin[i][1], lin[i][2], 0);
        check_linear(lin[i][0], lin[i][1], lin[i][2], 1);
    }

    static const int sp[][3] = {{1, 64, 16}, {3, 32, 5}, {9, 128, 33}, {16, 256, 48}};
    for (size_t i = 0; i < sizeof sp / sizeof sp[0]; i++) check_sparse(sp[i][0], sp[i][1], sp[i][2]);

    check_weight_rows(1, 1);
    check_weight_rows(5, 37);
    check_weight_rows(16, 256);

    static const int cv[][9] = {{1, 5, 5, 4, 3, 3, 1, 1, 1}, {2, 8, 7, 16, 8, 3, 2, 2, 1}, {1, 9, 9, 3, 5, 5, 4, 1, 2},
                                {3, 4, 6, 8, 4, 1, 0, 1, 1}, {1, 3, 3, 2, 2, 3, 0, 1, 1}, {1, 12, 10, 5, 7, 2, 0, 2, 3}};
    for (size_t i = 0; i < sizeof cv / sizeof cv[0]; i++)
        check_conv(cv[i][0], cv[i][1], cv[i][2], cv[i][3], cv[i][4], cv[i][5], cv[i][6], cv[i][7], cv[i][8]);

    static const int dw[][9] = {{1, 3, 9, 11, 3, 1, 1, 1, 1}, {2, 4, 8, 8, 5, 2, 2, 1, 0}, {1, 2, 7, 9, 3, 2, 1, 2, 1},
                                {1, 5, 6, 6, 1, 0, 1, 1, 0}, {1, 1, 4, 5, 7, 4, 3, 1, 1}};
    for (size_t i = 0; i < sizeof dw / sizeof dw[0]; i++)
        check_depthwise(dw[i][0], dw[i][1], dw[i][2], dw[i][3], dw[i][4], dw[i][5], dw[i][6], dw[i][7], dw[i][8]);

    check_convt(1, 3, 5, 7, 2, 1);
    check_convt(2, 16, 4, 4, 8, 0);

    orc_mt19937_t mt;
    orc_mt19937_seed(&mt, 5489u);
    uint32_t v = 0;
    for (int i = 0; i < 10000; i++) v = orc_mt19937_next(&mt);
    CHECK(v == 4123659995u, "mt19937 10000th output %u", v);

    if (g_fail) return 1;
    printf("oracle sanity: all checks passed\n");
    return 0;
}
