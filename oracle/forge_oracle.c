/*
 * forge_oracle.c -- CPU restatement of the reference's INT8 inference path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the thing measured or shipped):
 * loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
 * See forge_oracle.h for what pins each function.
 *
 * Arithmetic conventions (all IEEE-754 binary32, round-to-nearest-even):
 *   - quantize: scale = fmaxf(amax, 1e-8f) / 127.0f; inv = 1.0f / scale;
 *     q = clamp(rint(x * inv), -128, 127). IEEE division, as in the reference's host
 *     oracles (tests/test_quantize.cu:34-36, tests/test_int8_sparse_gemm.cu:243,250-251);
 *     RNE as the kernel's __float2int_rn (src/quant/quantize.cu:56,125-126).
 *   - GEMM dequant epilogue: fmaf((float)acc, as * ws, bias) then fp16 RNE
 *     (src/gemm/int8_dense.cu:171-174; src/gemm/int8_sparse.cu:659-661), i.e. the
 *     contracted form nvcc emits for `val *= as*ws; val += b`.
 *   - standalone dequant: fmaf((float)acc * as, ws, bias) (src/quant/dequantize.cu:22-26).
 */
#include "forge_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ------------------------------------------------------------------------- */
/* binary16 <-> binary32 (IEEE-754 semantics restated from the format)        */
/* ------------------------------------------------------------------------- */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_f16_to_f32(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1Fu;
    const uint32_t man = h & 0x3FFu;
    if (exp == 0x1F)                       /* inf / nan */
        return u2f(sign | 0x7F800000u | (man << 13));
    if (exp == 0) {
        if (man == 0) return u2f(sign);    /* +-0 */
        /* subnormal: man * 2^-24, exact in binary32 */
        const float v = (float)man * 5.9604644775390625e-08f;
        return (h & 0x8000u) ? -v : v;
    }
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

/* Round-to-nearest-even narrowing (the conversion __float2half performs). */
uint16_t orc_f32_to_f16(float f)
{
    const uint32_t u = f2u(f);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t abs = u & 0x7FFFFFFFu;
    if (abs > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((abs >> 13) & 0x3FFu)); /* nan */
    if (abs >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf */
    if (abs < 0x38800000u) {
        /* result is subnormal or zero: value / 2^-24, rounded to an integer, RNE */
        if (abs < 0x33000000u) return sign;   /* < 2^-25: rounds to 0 (2^-25 ties to even 0) */
        const uint32_t e = abs >> 23;         /* biased exponent 102..112 */
        const uint32_t m = (abs & 0x7FFFFFu) | 0x800000u;
        const int shift = (int)(126 - e);     /* value = m * 2^(e-150); /2^-24 -> m >> (126-e) */
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    /* normal range: drop 13 mantissa bits with RNE; carries propagate into the exponent */
    uint32_t r = abs - 0x38000000u;           /* rebias exponent 127 -> 15 */
    const uint32_t rem = r & 0x1FFFu;
    r >>= 13;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

/* ------------------------------------------------------------------------- */
/* Per-token quantization                                                     */
/* src/quant/quantize.cu:18-58 (two-pass) and :81-131 (vector); both compute  */
/* the same row absmax, scale and RNE quantization.                           */
/* ------------------------------------------------------------------------- */

void orc_quantize_rows(const uint16_t* x, int8_t* q, float* scales, int M, int K)
{
    for (int m = 0; m < M; m++) {
        const uint16_t* row = x + (size_t)m * K;
        float amax = 0.0f;
        /* quantize.cu: amax = fmaxf(amax, fabsf(x)), run on the GPU, whose max returns the
         * other operand for a NaN of either kind. C's fmaxf returns NaN when an operand is a
         * signalling NaN (glibc follows IEEE 754-2008 maxNum), so the skip is written out. */
        for (int k = 0; k < K; k++) {
            const float a = fabsf(orc_f16_to_f32(row[k]));
            if (a > amax) amax = a;
        }
        const float scale = fmaxf(amax, 1e-8f) / 127.0f;          /* quantize.cu:49,112 */
        const float inv = 1.0f / scale;                            /* quantize.cu:51,114 */
        scales[m] = scale;
        for (int k = 0; k < K; k++) {
            const float v = orc_f16_to_f32(row[k]) * inv;
            float r = rintf(v);                                    /* __float2int_rn: RNE */
            int qi;
            if (r != r) qi = 0;                                    /* NaN converts to 0 */
            else if (r < -128.0f) qi = -128;
            else if (r > 127.0f) qi = 127;
            else qi = (int)r;
            q[(size_t)m * K + k] = (int8_t)qi;                     /* clamp: quantize.cu:57 */
        }
    }
}

/* src/quant/dequantize.cu:22-26: val = (float)acc * as * ws (left to right), += bias. */
void orc_dequantize_bias(const int32_t* acc, const float* act_scale, const uint16_t* w_scale,
                         const uint16_t* bias, uint16_t* out, int M, int N)
{
    for (int m = 0; m < M; m++) {
        const float as = act_scale[m];
        for (int n = 0; n < N; n++) {
            const float p = (float)acc[(size_t)m * N + n] * as;
            const float ws = orc_f16_to_f32(w_scale[n]);
            const float v = bias ? fmaf(p, ws, orc_f16_to_f32(bias[n])) : p * ws;
            out[(size_t)m * N + n] = orc_f32_to_f16(v);
        }
    }
}

/* Split-K finalize, src/gemm/int8_sparse.cu:99-111: out = half(ws [+ float(bias[n])]), one
 * fp32 addition then fp16 RNE. */
void orc_splitk_reduce(const float* ws, const uint16_t* bias, uint16_t* out, int M, int N)
{
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float v = ws[(size_t)m * N + n];
            if (bias) v += orc_f16_to_f32(bias[n]);
            out[(size_t)m * N + n] = orc_f32_to_f16(v);
        }
}

/* ------------------------------------------------------------------------- */
/* Dense INT8 GEMM, C = A (M,K) x B (N,K)^T with INT32 accumulation           */
/* tests/test_int8_dense_gemm.cu:35-39; tests/test_int8_dp4a_gemm.cu:15-30    */
/* ------------------------------------------------------------------------- */

void orc_gemm_s32_rows(const int8_t* A, const int8_t* B, int32_t* C, int m0, int m1, int K, int N)
{
    for (int m = m0; m < m1; m++) {
        const int8_t* a = A + (size_t)m * K;
        for (int n = 0; n < N; n++) {
            const int8_t* b = B + (size_t)n * K;
            int32_t acc = 0;
            for (int k = 0; k < K; k++) acc += (int32_t)a[k] * (int32_t)b[k];
            C[(size_t)m * N + n] = acc;
        }
    }
}

void orc_gemm_s32(const int8_t* A, const int8_t* B, int32_t* C, int M, int K, int N)
{
    orc_gemm_s32_rows(A, B, C, 0, M, K, N);
}

/* Epilogue of src/gemm/int8_dense.cu:171-174 and src/gemm/int8_sparse.cu:659-661:
 * out = half(fmaf((float)acc, as*ws, bias)); without bias half((float)acc * (as*ws)). */
void orc_dequant_epilogue(const int32_t* acc, const float* act_scale, const uint16_t* w_scale,
                          const uint16_t* bias, uint16_t* out, int M, int N)
{
    for (int m = 0; m < M; m++) {
        for (int n = 0; n < N; n++) {
            const float s = act_scale[m] * orc_f16_to_f32(w_scale[n]);
            const float a = (float)acc[(size_t)m * N + n];
            const float v = bias ? fmaf(a, s, orc_f16_to_f32(bias[n])) : a * s;
            out[(size_t)m * N + n] = orc_f32_to_f16(v);
        }
    }
}

void orc_gemm_dequant(const int8_t* A, const int8_t* B, const float* act_scale,
                      const uint16_t* w_scale, const uint16_t* bias, uint16_t* out,
                      int M, int K, int N)
{
    int32_t* acc = (int32_t*)malloc((size_t)M * N * sizeof(int32_t));
    orc_gemm_s32(A, B, acc, M, K, N);
    orc_dequant_epilogue(acc, act_scale, w_scale, bias, out, M, N);
    free(acc);
}

/* src/gemm/int8_dense.cu:213-232: quantize x, then the dequantizing GEMM. */
void orc_linear(const uint16_t* x, const int8_t* W, const uint16_t* w_scale,
                const uint16_t* bias, uint16_t* out, int M, int K, int N)
{
    int8_t* q = (int8_t*)malloc((size_t)M * K);
    float* s = (float*)malloc((size_t)M * sizeof(float));
    orc_quantize_rows(x, q, s, M, K);
    orc_gemm_dequant(q, W, s, w_scale, bias, out, M, K, N);
    free(q);
    free(s);
}

/* ------------------------------------------------------------------------- */
/* 2:4 sparsity                                                               */
/* ------------------------------------------------------------------------- */

/* src/sparsity/prune_compress.cu:24-68. Per group of 4 along K: the two smallest
 * magnitudes are found with strict '<' comparisons seeded from positions (0,1), so
 * among equal magnitudes the lower index is pruned; the kept positions are stored
 * ascending with nibble keep0 | keep1 << 2. */
void orc_prune_compress_24(const int8_t* w, int8_t* comp, uint8_t* meta_raw, int N, int K)
{
    const int gpr = K / 4;
    for (int n = 0; n < N; n++) {
        for (int g = 0; g < gpr; g++) {
            const int8_t* v = w + (size_t)n * K + (size_t)g * 4;
            int a[4];
            for (int i = 0; i < 4; i++) a[i] = abs((int)v[i]);
            int min1 = 0, min2 = 1;
            if (a[min1] > a[min2]) { min1 = 1; min2 = 0; }
            for (int i = 2; i < 4; i++) {
                if (a[i] < a[min1]) { min2 = min1; min1 = i; }
                else if (a[i] < a[min2]) { min2 = i; }
            }
            int keep[2], kc = 0;
            for (int i = 0; i < 4; i++)
                if (i != min1 && i != min2) keep[kc++] = i;
            comp[(size_t)n * (K / 2) + (size_t)g * 2 + 0] = v[keep[0]];
            comp[(size_t)n * (K / 2) + (size_t)g * 2 + 1] = v[keep[1]];
            meta_raw[(size_t)n * gpr + g] = (uint8_t)(keep[0] | (keep[1] << 2));
        }
    }
}

/* Inverse of the compression (tests/test_prune_compress.cu:88-101 round trip). */
void orc_decompress_24(const int8_t* comp, const uint8_t* meta_raw, int8_t* w, int N, int K)
{
    const int gpr = K / 4;
    memset(w, 0, (size_t)N * K);
    for (int n = 0; n < N; n++) {
        for (int g = 0; g < gpr; g++) {
            const uint8_t nib = meta_raw[(size_t)n * gpr + g];
            const int k0 = nib & 3, k1 = (nib >> 2) & 3;
            int8_t* dst = w + (size_t)n * K + (size_t)g * 4;
            /* the second value wins if both indices coincide (never produced by pruning) */
            dst[k0] = comp[(size_t)n * (K / 2) + (size_t)g * 2 + 0];
            dst[k1] = comp[(size_t)n * (K / 2) + (size_t)g * 2 + 1];
        }
    }
}

/* src/sparsity/pack_metadata.cu:23-29: word (n, c) = sum_g nib[n, 8c+g] << 4g. */
void orc_pack_metadata_ref(const uint8_t* meta_raw, uint32_t* packed, int N, int K)
{
    const int gpr = K / 4, cpr = K / 32;
    for (int n = 0; n < N; n++)
        for (int c = 0; c < cpr; c++) {
            uint32_t p = 0;
            for (int g = 0; g < 8; g++)
                p |= ((uint32_t)(meta_raw[(size_t)n * gpr + c * 8 + g] & 0xFu)) << (4 * g);
            packed[(size_t)n * cpr + c] = p;
        }
}

/* gfx950 layout (this build's own format, same (N, K/32) uint32 size as the
 * reference): the reference word (n, c) is stored at
 *     (n / 16) * (K/32) * 16 + c * R + (n % 16),  R = min(16, N - 16 * (n / 16))
 * so that the 64 lanes of one v_smfmac_i32_16x16x128_i8 (lane = row%16 + 16*chunk)
 * read their index words of a full 16-row block as one contiguous 256-byte run; a
 * ragged last block (N % 16 != 0) stays a bijection onto [0, N*K/32). */
static size_t gfx950_pos(int n, int c, int N, int cpr)
{
    const int blk = n / 16;
    const int rows = (N - 16 * blk) < 16 ? (N - 16 * blk) : 16;
    return (size_t)blk * (size_t)cpr * 16 + (size_t)c * (size_t)rows + (size_t)(n % 16);
}

void orc_pack_metadata_gfx950(const uint8_t* meta_raw, uint32_t* packed, int N, int K)
{
    const int gpr = K / 4, cpr = K / 32;
    for (int n = 0; n < N; n++)
        for (int c = 0; c < cpr; c++) {
            uint32_t p = 0;
            for (int g = 0; g < 8; g++)
                p |= ((uint32_t)(meta_raw[(size_t)n * gpr + c * 8 + g] & 0xFu)) << (4 * g);
            packed[gfx950_pos(n, c, N, cpr)] = p;
        }
}

void orc_unpack_metadata_gfx950(const uint32_t* packed, uint8_t* meta_raw, int N, int K)
{
    const int gpr = K / 4, cpr = K / 32;
    for (int n = 0; n < N; n++)
        for (int c = 0; c < cpr; c++) {
            const uint32_t p = packed[gfx950_pos(n, c, N, cpr)];
            for (int g = 0; g < 8; g++)
                meta_raw[(size_t)n * gpr + c * 8 + g] = (uint8_t)((p >> (4 * g)) & 0xFu);
        }
}

/* Sparse GEMM, C (M, N) = x (M,K) x decompress(W_comp, meta)^T, INT32 accumulation:
 * the mathematical content of src/gemm/int8_sparse.cu:116-120 (before the epilogue),
 * restated as tests/test_int8_sparse_gemm.cu:65-81 does (GEMM of the pruned weights). */
void orc_sparse_gemm_s32(const int8_t* W_comp, const int8_t* x, const uint8_t* meta_raw,
                         int32_t* C, int M, int K, int N)
{
    int8_t* wd = (int8_t*)malloc((size_t)N * K);
    orc_decompress_24(W_comp, meta_raw, wd, N, K);
    orc_gemm_s32(x, wd, C, M, K, N);
    free(wd);
}

/* ------------------------------------------------------------------------- */
/* INT8 conv2d, NHWC input, OHWI weights, INT32 accumulation                 */
/* Index math from src/nn/int8_conv2d.cu:29-31 (conv_out_size) and :59-75.   */
/* ------------------------------------------------------------------------- */

int orc_conv_out_size(int in, int pad, int dil, int k, int stride)
{
    return (in + 2 * pad - dil * (k - 1) - 1) / stride + 1;
}

/* Output pixel rows r0 <= r < r1 (r = n * Ho + ho) of the direct convolution. */
static void conv2d_nhwc_s32_rows(const int8_t* x, const int8_t* w, int32_t* out,
                                 int H, int W, int C, int Co, int kH, int kW,
                                 int padH, int padW, int strideH, int strideW, int dilH, int dilW,
                                 int Ho, int Wo, int r0, int r1)
{
    for (int r = r0; r < r1; r++) {
        const int n = r / Ho, ho = r % Ho;
        for (int wo = 0; wo < Wo; wo++)
            for (int co = 0; co < Co; co++) {
                int32_t acc = 0;
                for (int kh = 0; kh < kH; kh++) {
                    const int hi = ho * strideH + kh * dilH - padH;
                    if (hi < 0 || hi >= H) continue;
                    for (int kw = 0; kw < kW; kw++) {
                        const int wi = wo * strideW + kw * dilW - padW;
                        if (wi < 0 || wi >= W) continue;
                        const int8_t* xp = x + (((size_t)n * H + hi) * W + wi) * C;
                        const int8_t* wp = w + (((size_t)co * kH + kh) * kW + kw) * C;
                        for (int c = 0; c < C; c++) acc += (int32_t)xp[c] * (int32_t)wp[c];
                    }
                }
                out[(((size_t)n * Ho + ho) * Wo + wo) * Co + co] = acc;
            }
    }
}

void orc_conv2d_nhwc_s32(const int8_t* x, const int8_t* w, int32_t* out,
                         int N, int H, int W, int C, int Co, int kH, int kW,
                         int padH, int padW, int strideH, int strideW, int dilH, int dilW)
{
    const int Ho = orc_conv_out_size(H, padH, dilH, kH, strideH);
    const int Wo = orc_conv_out_size(W, padW, dilW, kW, strideW);
    if (Ho <= 0 || Wo <= 0) return;
    conv2d_nhwc_s32_rows(x, w, out, H, W, C, Co, kH, kW, padH, padW, strideH, strideW, dilH, dilW,
                         Ho, Wo, 0, N * Ho);
}

/* ------------------------------------------------------------------------- */
/* Per-row symmetric weight quantization, python/forge/nn/linear.py:168-173    */
/* and :235-238 (torch float32 ops): scale = clamp(amax|w|, min=1e-8) / 127,   */
/* q = clamp(round(w / scale), -127, 127) with IEEE division and round half    */
/* to even, stored scale = scale.to(float16) (RNE). w is fp32 (the reference   */
/* converts any input to float32 first). Finite weights only: torch's amax and */
/* clamp propagate NaN and its float->int8 conversion of NaN is unspecified.   */
/* ------------------------------------------------------------------------- */

void orc_quantize_weight_rows(const float* w, int8_t* q, uint16_t* scale16, float* scale32, int N, int K)
{
    for (int n = 0; n < N; n++) {
        const float* row = w + (size_t)n * K;
        float amax = 0.0f;
        for (int k = 0; k < K; k++) amax = fmaxf(amax, fabsf(row[k]));
        const float scale = fmaxf(amax, 1e-8f) / 127.0f;
        for (int k = 0; k < K; k++) {
            float r = rintf(row[k] / scale);
            r = fminf(fmaxf(r, -127.0f), 127.0f);
            q[(size_t)n * K + k] = (int8_t)r;
        }
        if (scale16) scale16[n] = orc_f32_to_f16(scale);
        if (scale32) scale32[n] = scale;
    }
}

/* ------------------------------------------------------------------------- */
/* INT8 depthwise conv2d, NCHW FP16 in and out                               */
/* src/nn/int8_depthwise_conv2d.cu:25-70: per output, taps in (kh, kw) order, */
/* out-of-image taps skipped, w = (float)q * scale (one rounded product),     */
/* sum += inp * w as nvcc contracts it by default (-fmad=true): one fmaf per  */
/* tap from sum = +0; then sum + bias (when given) and fp16 RNE. The inputs   */
/* are fp16 and the scales fp16, so no fp32 denormal arises and the kernel's  */
/* fast-math flush-to-zero does not change a result.                          */
/* ------------------------------------------------------------------------- */

void orc_depthwise_conv2d(const uint16_t* in, const int8_t* w, const uint16_t* w_scale,
                          const uint16_t* bias, uint16_t* out, int N, int C, int H, int W,
                          int kH, int kW, int padH, int padW, int strideH, int strideW,
                          int dilH, int dilW)
{
    const int Ho = orc_conv_out_size(H, padH, dilH, kH, strideH);
    const int Wo = orc_conv_out_size(W, padW, dilW, kW, strideW);
    if (Ho <= 0 || Wo <= 0) return;
    for (int n = 0; n < N; n++)
        for (int c = 0; c < C; c++) {
            const float scale = orc_f16_to_f32(w_scale[c]);
            const int8_t* wc = w + (size_t)c * kH * kW;
            const uint16_t* x = in + ((size_t)n * C + c) * H * W;
            uint16_t* y = out + ((size_t)n * C + c) * Ho * Wo;
            for (int ho = 0; ho < Ho; ho++)
                for (int wo = 0; wo < Wo; wo++) {
                    float sum = 0.0f;
                    for (int kh = 0; kh < kH; kh++) {
                        const int hi = ho * strideH + kh * dilH - padH;
                        if (hi < 0 || hi >= H) continue;
                        for (int kw = 0; kw < kW; kw++) {
                            const int wi = wo * strideW + kw * dilW - padW;
                            if (wi < 0 || wi >= W) continue;
                            const float wf = (float)wc[kh * kW + kw] * scale;
                            sum = fmaf(orc_f16_to_f32(x[(size_t)hi * W + wi]), wf, sum);
                        }
                    }
                    if (bias) sum = sum + orc_f16_to_f32(bias[c]);
                    y[(size_t)ho * Wo + wo] = orc_f32_to_f16(sum);
                }
        }
}

/* ------------------------------------------------------------------------- */
/* INT8 ConvTranspose2d, kernel 2, stride 2, NCHW FP16 in and out             */
/* src/nn/int8_conv_transpose2d.cu:128-191. Per image: pixel p's channel      */
/* vector x[:, p] is quantized as one row (quantize.cu arithmetic, above);    */
/* GEMM row p against weight rows n = co*4 + kh*2 + kw (repacked (4*C_out,    */
/* C_in)); the GEMM epilogue runs without bias with w_scale replicated per    */
/* co (:50-60, :174-181): g = half((float)acc * (as * ws[co])); the scatter   */
/* (:70-102) writes out[co, 2h+kh, 2w+kw] = half((float)g + bias[co]), or g   */
/* unchanged without bias. acc32 (optional) receives the INT32 GEMM stage in  */
/* the output's NCHW layout.                                                  */
/* ------------------------------------------------------------------------- */

void orc_conv_transpose2d_k2s2(const uint16_t* in, const int8_t* w, const uint16_t* w_scale,
                               const uint16_t* bias, uint16_t* out, int32_t* acc32,
                               int N, int C_in, int H, int W, int C_out)
{
    const size_t HW = (size_t)H * W;
    const int Ng = 4 * C_out;
    uint16_t* col = (uint16_t*)malloc((size_t)C_in * sizeof(uint16_t));
    int8_t* q = (int8_t*)malloc((size_t)C_in);
    for (int n = 0; n < N; n++) {
        const uint16_t* x = in + (size_t)n * C_in * HW;
        for (size_t p = 0; p < HW; p++) {
            const int h = (int)(p / W), wi = (int)(p % W);
            for (int ci = 0; ci < C_in; ci++) col[ci] = x[(size_t)ci * HW + p];
            float as;
            orc_quantize_rows(col, q, &as, 1, C_in);
            for (int j = 0; j < Ng; j++) {
                const int8_t* wr = w + (size_t)j * C_in;
                int32_t acc = 0;
                for (int ci = 0; ci < C_in; ci++) acc += (int32_t)q[ci] * (int32_t)wr[ci];
                const int co = j >> 2, kh = (j >> 1) & 1, kw = j & 1;
                const float s = as * orc_f16_to_f32(w_scale[co]);
                uint16_t g = orc_f32_to_f16((float)acc * s);
                if (bias) g = orc_f32_to_f16(orc_f16_to_f32(g) + orc_f16_to_f32(bias[co]));
                const size_t o = (((size_t)n * C_out + co) * 2 * H + 2 * h + kh) * (size_t)(2 * W) + 2 * wi + kw;
                if (out) out[o] = g;
                if (acc32) acc32[o] = acc;
            }
        }
    }
    free(col);
    free(q);
}

/* ------------------------------------------------------------------------- */
/* MT19937 (Matsumoto & Nishimura 1998), as std::mt19937 specifies it.        */
/* Used to regenerate the reference test's pack_metadata input vectors        */
/* (tests/test_pack_metadata.cu:124-126: std::mt19937 rng(42); rng() & 0xF).  */
/* ------------------------------------------------------------------------- */

void orc_mt19937_seed(orc_mt19937_t* s, uint32_t seed)
{
    s->mt[0] = seed;
    for (int i = 1; i < 624; i++)
        s->mt[i] = 1812433253u * (s->mt[i - 1] ^ (s->mt[i - 1] >> 30)) + (uint32_t)i;
    s->idx = 624;
}

uint32_t orc_mt19937_next(orc_mt19937_t* s)
{
    if (s->idx >= 624) {
        for (int i = 0; i < 624; i++) {
            const uint32_t y = (s->mt[i] & 0x80000000u) | (s->mt[(i + 1) % 624] & 0x7FFFFFFFu);
            s->mt[i] = s->mt[(i + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908B0DFu : 0u);
        }
        s->idx = 0;
    }
    uint32_t y = s->mt[s->idx++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9D2C5680u;
    y ^= (y << 15) & 0xEFC60000u;
    y ^= y >> 18;
    return y;
}

/* ------------------------------------------------------------------------- */
/* CPU baseline timing: the host INT32 loop plus the dequant epilogue over a  */
/* slice of rows, single-threaded. Returns seconds.                           */
/* ------------------------------------------------------------------------- */

/* The same work split over output rows on `threads` POSIX threads (the multi-core CPU
 * baseline: each thread runs the INT32 loop and the epilogue on a contiguous row range). */
typedef struct {
    const int8_t *A, *B;
    const float* act_scale;
    const uint16_t *w_scale, *bias;
    uint16_t* out;
    int32_t* acc;
    int r0, r1, K, N;
} orc_rows_job;

static void* orc_rows_worker(void* p)
{
    const orc_rows_job* j = (const orc_rows_job*)p;
    if (j->r1 > j->r0) {
        orc_gemm_s32_rows(j->A, j->B, j->acc, j->r0, j->r1, j->K, j->N);
        orc_dequant_epilogue(j->acc + (size_t)j->r0 * j->N, j->act_scale + j->r0, j->w_scale, j->bias,
                             j->out + (size_t)j->r0 * j->N, j->r1 - j->r0, j->N);
    }
    return NULL;
}

double orc_time_gemm_dequant_rows_mt(const int8_t* A, const int8_t* B, const float* act_scale,
                                     const uint16_t* w_scale, const uint16_t* bias, uint16_t* out,
                                     int rows, int K, int N, int threads)
{
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    struct timespec t0, t1;
    int32_t* acc = (int32_t*)malloc((size_t)rows * N * sizeof(int32_t));
    pthread_t tid[256];
    orc_rows_job jobs[256];
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (int t = 0; t < threads; t++) {
        const orc_rows_job j = {A, B, act_scale, w_scale, bias, out, acc,
                                (int)((long long)rows * t / threads), (int)((long long)rows * (t + 1) / threads), K, N};
        jobs[t] = j;
        pthread_create(&tid[t], NULL, orc_rows_worker, &jobs[t]);
    }
    for (int t = 0; t < threads; t++) pthread_join(tid[t], NULL);
    clock_gettime(CLOCK_MONOTONIC, &t1);
    free(acc);
    return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}

double orc_time_gemm_dequant_rows(const int8_t* A, const int8_t* B, const float* act_scale,
                                  const uint16_t* w_scale, const uint16_t* bias, uint16_t* out,
                                  int rows, int K, int N)
{
    struct timespec t0, t1;
    int32_t* acc = (int32_t*)malloc((size_t)rows * N * sizeof(int32_t));
    clock_gettime(CLOCK_MONOTONIC, &t0);
    orc_gemm_s32_rows(A, B, acc, 0, rows, K, N);
    orc_dequant_epilogue(acc, act_scale, w_scale, bias, out, rows, N);
    clock_gettime(CLOCK_MONOTONIC, &t1);
    free(acc);
    return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}

/* ------------------------------------------------------------------------- */
/* Threaded forms of the GEMM and conv loops (for whole-output comparisons at  */
/* full size). Each thread runs the single-threaded code on a contiguous range */
/* of output rows, so every output has the same bits as the plain function.    */
/* ------------------------------------------------------------------------- */

typedef struct {
    int kind; /* 0 gemm_s32, 1 gemm_dequant, 2 conv */
    const int8_t *A, *B;
    const float* act_scale;
    const uint16_t *w_scale, *bias;
    uint16_t* out16;
    int32_t* C;
    int r0, r1, K, N;
    /* conv geometry */
    int H, W, Cc, Co, kH, kW, padH, padW, sH, sW, dH, dW, Ho, Wo;
} orc_range_job;

static void* orc_range_worker(void* p)
{
    const orc_range_job* j = (const orc_range_job*)p;
    if (j->r1 <= j->r0) return NULL;
    if (j->kind == 2) {
        conv2d_nhwc_s32_rows(j->A, j->B, j->C, j->H, j->W, j->Cc, j->Co, j->kH, j->kW, j->padH, j->padW,
                             j->sH, j->sW, j->dH, j->dW, j->Ho, j->Wo, j->r0, j->r1);
        return NULL;
    }
    orc_gemm_s32_rows(j->A, j->B, j->C, j->r0, j->r1, j->K, j->N);
    if (j->kind == 1)
        orc_dequant_epilogue(j->C + (size_t)j->r0 * j->N, j->act_scale + j->r0, j->w_scale, j->bias,
                             j->out16 + (size_t)j->r0 * j->N, j->r1 - j->r0, j->N);
    return NULL;
}

static void orc_run_rows(const orc_range_job* proto, int rows, int threads)
{
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    if (threads > rows) threads = rows > 0 ? rows : 1;
    pthread_t tid[256];
    orc_range_job jobs[256];
    int started[256];
    for (int t = 0; t < threads; t++) {
        jobs[t] = *proto;
        jobs[t].r0 = (int)((long long)rows * t / threads);
        jobs[t].r1 = (int)((long long)rows * (t + 1) / threads);
        started[t] = pthread_create(&tid[t], NULL, orc_range_worker, &jobs[t]) == 0;
        if (!started[t]) orc_range_worker(&jobs[t]);   /* no thread: run the range here */
    }
    for (int t = 0; t < threads; t++)
        if (started[t]) pthread_join(tid[t], NULL);
}

void orc_gemm_s32_mt(const int8_t* A, const int8_t* B, int32_t* C, int M, int K, int N, int threads)
{
    orc_range_job j;
    memset(&j, 0, sizeof j);
    j.kind = 0; j.A = A; j.B = B; j.C = C; j.K = K; j.N = N;
    orc_run_rows(&j, M, threads);
}

void orc_gemm_dequant_mt(const int8_t* A, const int8_t* B, const float* act_scale,
                         const uint16_t* w_scale, const uint16_t* bias, uint16_t* out,
                         int M, int K, int N, int threads)
{
    int32_t* acc = (int32_t*)malloc((size_t)M * N * sizeof(int32_t));
    orc_range_job j;
    memset(&j, 0, sizeof j);
    j.kind = 1; j.A = A; j.B = B; j.C = acc; j.K = K; j.N = N;
    j.act_scale = act_scale; j.w_scale = w_scale; j.bias = bias; j.out16 = out;
    orc_run_rows(&j, M, threads);
    free(acc);
}

void orc_sparse_gemm_s32_mt(const int8_t* W_comp, const int8_t* x, const uint8_t* meta_raw,
                            int32_t* C, int M, int K, int N, int threads)
{
    int8_t* wd = (int8_t*)malloc((size_t)N * K);
    orc_decompress_24(W_comp, meta_raw, wd, N, K);
    orc_gemm_s32_mt(x, wd, C, M, K, N, threads);
    free(wd);
}

void orc_conv2d_nhwc_s32_mt(const int8_t* x, const int8_t* w, int32_t* out,
                            int N, int H, int W, int C, int Co, int kH, int kW,
                            int padH, int padW, int strideH, int strideW, int dilH, int dilW, int threads)
{
    const int Ho = orc_conv_out_size(H, padH, dilH, kH, strideH);
    const int Wo = orc_conv_out_size(W, padW, dilW, kW, strideW);
    if (Ho <= 0 || Wo <= 0) return;
    orc_range_job j;
    memset(&j, 0, sizeof j);
    j.kind = 2; j.A = x; j.B = w; j.C = out;
    j.H = H; j.W = W; j.Cc = C; j.Co = Co; j.kH = kH; j.kW = kW; j.padH = padH; j.padW = padW;
    j.sH = strideH; j.sW = strideW; j.dH = dilH; j.dW = dilW; j.Ho = Ho; j.Wo = Wo;
    orc_run_rows(&j, N * Ho, threads);
}
