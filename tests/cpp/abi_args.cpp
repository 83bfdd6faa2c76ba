// C-ABI argument checks under host AddressSanitizer + UndefinedBehaviorSanitizer, with no GPU.
//
// Test infrastructure (tests/cpp/build_san.py builds it against the host-sanitized library,
// tests/test_sanitizers.py runs it on the CPU). Every entry point of include/forge_amd.h is
// called with:
//   - empty shapes (a zero or negative M, N, K, C, H, W) and null pointers: FORGE_OK and no
//     work, as the reference's launchers return early;
//   - a null required operand at a valid shape: FORGE_EINVAL before any device call;
//   - shape-contract violations the header names (K % 64 for the sparse GEMM, K % 4 for
//     prune/compress, threads outside [1, 1024], strides or dilations <= 0, ...): FORGE_EINVAL;
//   - valid arguments (host buffers standing in for device memory): no device here, so a
//     non-zero status (FORGE_ENODEV or a HIP error), never a crash;
// and the host-only functions (plan, fused chooser, workspace sizes) over extreme sizes, where
// the sanitizers report any signed overflow, division by zero or out-of-bounds access.
// Prints one line per failed expectation; exit status 0 when there is none.
#include "forge_amd.h"

#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

static int g_fail = 0;

static void expect(bool ok, const char* what, int line) {
    if (!ok) {
        std::fprintf(stderr, "FAIL line %d: %s\n", line, what);
        g_fail = 1;
    }
}
#define EXPECT_EQ(call, want)                                                              \
    do {                                                                                   \
        const int got_ = (call);                                                           \
        if (got_ != (want)) {                                                              \
            std::fprintf(stderr, "FAIL line %d: %s = %d, want %d\n", __LINE__, #call, got_, \
                         static_cast<int>(want));                                          \
            g_fail = 1;                                                                    \
        }                                                                                  \
    } while (0)
#define EXPECT_ERR(call)                                                                   \
    do {                                                                                   \
        const int got_ = (call);                                                           \
        if (got_ == FORGE_OK) {                                                            \
            std::fprintf(stderr, "FAIL line %d: %s = FORGE_OK without a device\n", __LINE__, \
                         #call);                                                           \
            g_fail = 1;                                                                    \
        }                                                                                  \
    } while (0)

int main()
{
    // Host buffers big enough for every "valid" call below (never dereferenced without a device).
    std::vector<unsigned char> buf(1 << 20, 0);
    void* b = buf.data();
    auto u16 = static_cast<uint16_t*>(b);
    auto i8 = static_cast<int8_t*>(b);
    auto u8 = static_cast<uint8_t*>(b);
    auto i32 = static_cast<int32_t*>(b);
    auto u32 = static_cast<uint32_t*>(b);
    auto f32 = static_cast<float*>(b);
    void* st = nullptr;

    // ---- library ----
    for (int s : {FORGE_OK, FORGE_EINVAL, FORGE_ENODEV, FORGE_ERANGE, 1, 2, 98, 100, 1000, -4, -1000, INT_MAX, INT_MIN})
        expect(forge_status_string(s) != nullptr, "forge_status_string returns text", __LINE__);
    expect(std::strcmp(forge_last_route(), "none") == 0, "forge_last_route before any launch is \"none\"", __LINE__);
    EXPECT_EQ(forge_ksplit_last(nullptr, nullptr), FORGE_EINVAL);
    {
        int slot = 7, parts = 7;
        EXPECT_EQ(forge_ksplit_last(&slot, &parts), FORGE_OK);
        expect(slot == -1 && parts == 0, "forge_ksplit_last before any decode launch: slot -1, parts 0", __LINE__);
    }
    EXPECT_ERR(forge_init());
    EXPECT_ERR(forge_ksplit_reset(st));
    EXPECT_EQ(forge_slots_in_use(nullptr, nullptr, nullptr, nullptr), FORGE_EINVAL);
    {
        int a = 0, b2 = 0, c = 0, d = 0;
        EXPECT_EQ(forge_slots_in_use(&a, &b2, nullptr, &d), FORGE_EINVAL);
        EXPECT_ERR(forge_slots_in_use(&a, &b2, &c, &d));   // no device here
    }
    EXPECT_EQ(forge_get_compute_capability(0, nullptr), FORGE_EINVAL);
    EXPECT_EQ(forge_has_int8_matrix_cores(0, nullptr), FORGE_EINVAL);
    {
        int v = 0;
        EXPECT_ERR(forge_get_compute_capability(0, &v));
        EXPECT_ERR(forge_get_compute_capability(-1, &v));
        EXPECT_ERR(forge_has_int8_matrix_cores(INT_MAX, &v));
    }

    // ---- quantization ----
    EXPECT_EQ(forge_quantize_activation(nullptr, nullptr, nullptr, 0, 64, st), FORGE_OK);
    EXPECT_EQ(forge_quantize_activation(nullptr, nullptr, nullptr, 4, 0, st), FORGE_OK);
    EXPECT_EQ(forge_quantize_activation(nullptr, nullptr, nullptr, -3, 64, st), FORGE_OK);
    EXPECT_EQ(forge_quantize_activation(nullptr, i8, f32, 4, 64, st), FORGE_EINVAL);
    EXPECT_EQ(forge_quantize_activation(u16, nullptr, f32, 4, 64, st), FORGE_EINVAL);
    EXPECT_EQ(forge_quantize_activation(u16, i8, nullptr, 4, 64, st), FORGE_EINVAL);
    EXPECT_ERR(forge_quantize_activation(u16, i8, f32, 4, 64, st));
    EXPECT_EQ(forge_quantize_activation_twopass(nullptr, nullptr, nullptr, 0, 64, 256, st), FORGE_OK);
    EXPECT_EQ(forge_quantize_activation_twopass(nullptr, i8, f32, 4, 64, 256, st), FORGE_EINVAL);
    EXPECT_EQ(forge_quantize_activation_twopass(u16, i8, f32, 4, 64, 0, st), FORGE_EINVAL);
    EXPECT_EQ(forge_quantize_activation_twopass(u16, i8, f32, 4, 64, 1025, st), FORGE_EINVAL);
    EXPECT_EQ(forge_quantize_activation_twopass(u16, i8, f32, 4, 64, -5, st), FORGE_EINVAL);
    EXPECT_ERR(forge_quantize_activation_twopass(u16, i8, f32, 4, 64, 128, st));
    EXPECT_EQ(forge_dequantize_bias(nullptr, nullptr, nullptr, nullptr, nullptr, 0, 8, st), FORGE_OK);
    EXPECT_EQ(forge_dequantize_bias(nullptr, f32, u16, u16, u16, 4, 8, st), FORGE_EINVAL);
    EXPECT_EQ(forge_dequantize_bias(i32, nullptr, u16, u16, u16, 4, 8, st), FORGE_EINVAL);
    EXPECT_EQ(forge_dequantize_bias(i32, f32, nullptr, u16, u16, 4, 8, st), FORGE_EINVAL);
    EXPECT_EQ(forge_dequantize_bias(i32, f32, u16, u16, nullptr, 4, 8, st), FORGE_EINVAL);
    EXPECT_ERR(forge_dequantize_bias(i32, f32, u16, nullptr, u16, 4, 8, st));

    // ---- dense GEMM ----
    EXPECT_EQ(forge_int8_gemm_dequant(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0, 64, 64, st), FORGE_OK);
    EXPECT_EQ(forge_int8_gemm_dequant(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 64, -1, 64, st), FORGE_OK);
    EXPECT_EQ(forge_int8_gemm_dequant(nullptr, i8, f32, u16, u16, u16, 64, 64, 64, st), FORGE_EINVAL);
    EXPECT_EQ(forge_int8_gemm_dequant(i8, nullptr, f32, u16, u16, u16, 64, 64, 64, st), FORGE_EINVAL);
    EXPECT_EQ(forge_int8_gemm_dequant(i8, i8, nullptr, u16, u16, u16, 64, 64, 64, st), FORGE_EINVAL);
    EXPECT_EQ(forge_int8_gemm_dequant(i8, i8, f32, nullptr, u16, u16, 64, 64, 64, st), FORGE_EINVAL);
    EXPECT_EQ(forge_int8_gemm_dequant(i8, i8, f32, u16, u16, nullptr, 64, 64, 64, st), FORGE_EINVAL);
    EXPECT_ERR(forge_int8_gemm_dequant(i8, i8, f32, u16, nullptr, u16, 64, 64, 64, st));
    EXPECT_EQ(forge_int8_gemm(nullptr, i8, f32, u16, u16, u16, 64, 64, 64, st), FORGE_EINVAL);
    EXPECT_ERR(forge_int8_gemm(i8, i8, f32, u16, u16, u16, 1, 128, 16, st));
    EXPECT_EQ(forge_int8_gemm_s32(nullptr, nullptr, nullptr, 64, 64, 0, st), FORGE_OK);
    EXPECT_EQ(forge_int8_gemm_s32(i8, i8, nullptr, 64, 64, 64, st), FORGE_EINVAL);
    EXPECT_ERR(forge_int8_gemm_s32(i8, i8, i32, 4096, 4096, 4096, st));
    EXPECT_EQ(forge_int8_linear(nullptr, nullptr, nullptr, nullptr, nullptr, 0, 64, 64, nullptr, nullptr, st),
              FORGE_OK);
    EXPECT_EQ(forge_int8_linear(u16, i8, u16, u16, u16, 16, 64, 64, nullptr, f32, st), FORGE_EINVAL);
    EXPECT_EQ(forge_int8_linear(u16, i8, u16, u16, u16, 16, 64, 64, i8, nullptr, st), FORGE_EINVAL);
    EXPECT_EQ(forge_int8_linear(u16, nullptr, u16, u16, u16, 16, 64, 64, i8, f32, st), FORGE_EINVAL);
    EXPECT_ERR(forge_int8_linear(u16, i8, u16, u16, u16, 1, 256, 64, i8, f32, st));
    EXPECT_ERR(forge_int8_linear(u16, i8, u16, u16, u16, 16, 8192, 8192, i8, f32, st));
    EXPECT_EQ(forge_int8_linear_noalloc(nullptr, nullptr, nullptr, nullptr, nullptr, 0, 64, 64, st), FORGE_OK);
    EXPECT_EQ(forge_int8_linear_noalloc(u16, nullptr, u16, u16, u16, 16, 64, 64, st), FORGE_EINVAL);
    EXPECT_EQ(forge_int8_linear_noalloc(u16, i8, u16, u16, u16, 65537, 64, 64, st), FORGE_ERANGE);
    EXPECT_EQ(forge_int8_linear_noalloc(u16, i8, u16, u16, u16, 4096, 8192, 64, st), FORGE_ERANGE);
    EXPECT_EQ(forge_int8_linear_noalloc(u16, i8, u16, u16, u16, INT_MAX, INT_MAX, 64, st), FORGE_ERANGE);
    EXPECT_ERR(forge_int8_linear_noalloc(u16, i8, u16, u16, u16, 16, 64, 64, st));

    // ---- 2:4 sparsity ----
    EXPECT_EQ(forge_prune_compress_24(nullptr, nullptr, nullptr, 0, 64, st), FORGE_OK);
    EXPECT_EQ(forge_prune_compress_24(nullptr, i8, u8, 16, 64, st), FORGE_EINVAL);
    EXPECT_EQ(forge_prune_compress_24(i8, i8, u8, 16, 66, st), FORGE_EINVAL);
    EXPECT_ERR(forge_prune_compress_24(i8, i8, u8, 16, 64, st));
    EXPECT_EQ(forge_pack_metadata(nullptr, nullptr, 0, 64, st), FORGE_OK);
    EXPECT_EQ(forge_pack_metadata(nullptr, u32, 16, 64, st), FORGE_EINVAL);
    EXPECT_EQ(forge_pack_metadata(u8, u32, 16, 48, st), FORGE_EINVAL);
    EXPECT_ERR(forge_pack_metadata(u8, u32, 16, 64, st));
    EXPECT_EQ(forge_unpack_metadata(nullptr, nullptr, 0, 64, st), FORGE_OK);
    EXPECT_EQ(forge_unpack_metadata(u32, nullptr, 16, 64, st), FORGE_EINVAL);
    EXPECT_EQ(forge_unpack_metadata(u32, u8, 16, 40, st), FORGE_EINVAL);
    EXPECT_ERR(forge_unpack_metadata(u32, u8, 16, 64, st));

    // ---- sparse GEMM: the planner and the chooser are host arithmetic ----
    {
        int tile = -7, split = -7;
        EXPECT_EQ(forge_sparse_int8_gemm_plan(64, 64, 64, 0, 1, FORGE_SPARSE_TILE_AUTO, nullptr, &split), FORGE_EINVAL);
        EXPECT_EQ(forge_sparse_int8_gemm_plan(64, 64, 64, 0, 1, FORGE_SPARSE_TILE_AUTO, &tile, nullptr), FORGE_EINVAL);
        // a tile index outside 0..2 means the automatic choice (int8_sparse.cu:897, :907)
        int tile_auto = -7, split_auto = -7;
        EXPECT_EQ(forge_sparse_int8_gemm_plan(4096, 4096, 4096, 0, 1, FORGE_SPARSE_TILE_AUTO, &tile_auto, &split_auto),
                  FORGE_OK);
        EXPECT_EQ(forge_sparse_int8_gemm_plan(4096, 4096, 4096, 0, 1, 3, &tile, &split), FORGE_OK);
        expect(tile == tile_auto && split == split_auto, "plan: tile 3 is the automatic choice", __LINE__);
        EXPECT_EQ(forge_sparse_int8_gemm_plan(4096, 4096, 4096, 0, 1, -2, &tile, &split), FORGE_OK);
        expect(tile == tile_auto && split == split_auto, "plan: tile -2 is the automatic choice", __LINE__);
        const int sizes[] = {0, 1, 15, 16, 63, 64, 65, 127, 1024, 4096, 11008, 65536, 1 << 20, INT_MAX / 2, INT_MAX - 1,
                             INT_MAX, -1, INT_MIN};
        for (int M : sizes)
            for (int K : sizes)
                for (int N : sizes)
                    for (int sk : {0, 1, 3, 64, INT_MAX, -1})
                        for (int ws : {0, 1}) {
                            tile = split = -7;
                            const int r = forge_sparse_int8_gemm_plan(M, K, N, sk, ws, FORGE_SPARSE_TILE_AUTO, &tile,
                                                                      &split);
                            if (r == FORGE_OK)
                                expect(tile >= 0 && tile < FORGE_SPARSE_NUM_TILES && split >= 1 && (ws || split == 1),
                                       "plan: tile in range, split >= 1, no split without a workspace", __LINE__);
                            int flag = -1;
                            const int f = forge_sparse_int8_linear_fused(M, K, N, &flag);
                            if (f == FORGE_OK) expect(flag == 0 || flag == 1, "fused chooser flag is 0 or 1", __LINE__);
                        }
        EXPECT_EQ(forge_sparse_int8_linear_fused(64, 64, 64, nullptr), FORGE_EINVAL);
    }
    EXPECT_EQ(forge_sparse_int8_gemm(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0, 64, 64, nullptr,
                                     1, st, FORGE_SPARSE_TILE_AUTO),
              FORGE_OK);
    EXPECT_EQ(forge_sparse_int8_gemm(nullptr, i8, u32, f32, u16, u16, u16, 16, 64, 64, nullptr, 1, st, -1), FORGE_EINVAL);
    EXPECT_EQ(forge_sparse_int8_gemm(i8, i8, u32, f32, u16, u16, u16, 16, 96, 64, nullptr, 1, st, -1), FORGE_EINVAL);
    EXPECT_EQ(forge_sparse_int8_gemm(i8, i8, u32, f32, u16, u16, u16, 16, 64, 24, nullptr, 1, st, -1), FORGE_EINVAL);
    EXPECT_ERR(forge_sparse_int8_gemm(i8, i8, u32, f32, u16, u16, u16, 16, 64, 64, nullptr, 1, st, 5));
    EXPECT_ERR(forge_sparse_int8_gemm(i8, i8, u32, f32, u16, u16, u16, 16, 64, 64, nullptr, 1, st, -1));
    EXPECT_EQ(forge_sparse_int8_gemm_s32(nullptr, nullptr, nullptr, nullptr, 16, 64, 0, st), FORGE_OK);
    EXPECT_EQ(forge_sparse_int8_gemm_s32(i8, i8, u32, nullptr, 16, 64, 64, st), FORGE_EINVAL);
    EXPECT_EQ(forge_sparse_int8_gemm_s32(i8, i8, u32, i32, 16, 32, 64, st), FORGE_EINVAL);
    EXPECT_ERR(forge_sparse_int8_gemm_s32(i8, i8, u32, i32, 16, 64, 64, st));
    EXPECT_EQ(forge_sparse_int8_linear(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0, 64, 64, nullptr, nullptr,
                                       nullptr, 0, st, -1),
              FORGE_OK);
    EXPECT_EQ(forge_sparse_int8_linear(u16, i8, u32, u16, u16, u16, 16, 64, 64, nullptr, f32, nullptr, 0, st, -1),
              FORGE_EINVAL);
    // a path other than auto (-1) or fused (1) is the two-pass path (int8_sparse.cu:1027-1029)
    EXPECT_ERR(forge_sparse_int8_linear(u16, i8, u32, u16, u16, u16, 16, 64, 64, i8, f32, nullptr, 0, st, 2));
    EXPECT_EQ(forge_sparse_int8_linear(u16, i8, u32, u16, u16, u16, 16, 100, 64, i8, f32, nullptr, 0, st, -1),
              FORGE_EINVAL);
    EXPECT_ERR(forge_sparse_int8_linear(u16, i8, u32, u16, u16, u16, 16, 64, 64, i8, f32, nullptr, 0, st, -1));
    EXPECT_EQ(forge_splitk_reduce(nullptr, nullptr, nullptr, 0, 64, st), FORGE_OK);
    EXPECT_EQ(forge_splitk_reduce(nullptr, u16, u16, 16, 64, st), FORGE_EINVAL);
    EXPECT_EQ(forge_splitk_reduce(f32, u16, nullptr, 16, 64, st), FORGE_EINVAL);
    EXPECT_ERR(forge_splitk_reduce(f32, nullptr, u16, 16, 64, st));

    // ---- weight preparation ----
    EXPECT_EQ(forge_quantize_weight_rows(nullptr, 0, nullptr, nullptr, 0, 64, st), FORGE_OK);
    EXPECT_EQ(forge_quantize_weight_rows(nullptr, 0, i8, u16, 16, 64, st), FORGE_EINVAL);
    EXPECT_EQ(forge_quantize_weight_rows(f32, 0, i8, nullptr, 16, 64, st), FORGE_EINVAL);
    EXPECT_ERR(forge_quantize_weight_rows(f32, 1, i8, u16, 16, 64, st));
    EXPECT_EQ(forge_prepare_sparse_weight(nullptr, 0, nullptr, nullptr, nullptr, 0, 64, st), FORGE_OK);
    EXPECT_EQ(forge_prepare_sparse_weight(f32, 0, i8, nullptr, u16, 16, 64, st), FORGE_EINVAL);
    EXPECT_EQ(forge_prepare_sparse_weight(f32, 0, i8, u32, u16, 16, 48, st), FORGE_EINVAL);
    EXPECT_ERR(forge_prepare_sparse_weight(f32, 0, i8, u32, u16, 16, 64, st));

    // ---- convolutions ----
    // workspace sizes: 0 for any non-positive dimension or an empty output, never UB
    const int dims[] = {-1, 0, 1, 3, 64, 4096, 1 << 20, INT_MAX};
    for (int C : dims)
        for (int HW : dims)
            for (int Co : dims) {
                (void)forge_int8_conv_transpose2d_k2s2_workspace_size(C, HW, HW, Co);
                for (int k : {-1, 0, 1, 3, INT_MAX})
                    for (int s : {-1, 0, 1, 2, INT_MAX})
                        (void)forge_int8_conv2d_workspace_size(C, HW, HW, Co, k, k, 1, 1, s, s, 1, 1);
            }
    EXPECT_EQ(static_cast<int>(forge_int8_conv2d_workspace_size(16, 8, 8, 16, 3, 3, 1, 1, 0, 1, 1, 1)), 0);
    EXPECT_EQ(static_cast<int>(forge_int8_conv2d_workspace_size(16, 8, 8, 16, 3, 3, -1, 1, 1, 1, 1, 1)), 0);
    EXPECT_EQ(static_cast<int>(forge_int8_conv2d_workspace_size(16, 8, 8, 16, 3, 3, 1, 1, 1, 1, 0, 1)), 0);
    EXPECT_EQ(static_cast<int>(forge_int8_conv_transpose2d_k2s2_workspace_size(0, 8, 8, 16)), 0);

    EXPECT_EQ(forge_int8_conv2d_forward(nullptr, nullptr, nullptr, nullptr, nullptr, 0, 16, 8, 8, 16, 3, 3, 1, 1, 1, 1,
                                        1, 1, nullptr, st),
              FORGE_OK);
    EXPECT_EQ(forge_int8_conv2d_forward(u16, i8, u16, u16, u16, 1, 16, 8, 8, 16, 3, 3, 1, 1, 1, 1, 1, 1, nullptr, st),
              FORGE_EINVAL);
    EXPECT_EQ(forge_int8_conv2d_forward(u16, i8, u16, u16, u16, 1, 16, 8, 8, 16, 3, 3, 1, 1, 0, 1, 1, 1, b, st),
              FORGE_EINVAL);
    EXPECT_EQ(forge_int8_conv2d_forward(u16, i8, u16, u16, u16, 1, 16, 8, 8, 16, 3, 3, 1, 1, 1, -2, 1, 1, b, st),
              FORGE_EINVAL);
    EXPECT_EQ(forge_int8_conv2d_forward(u16, i8, u16, u16, u16, 1, 16, 8, 8, 16, 3, 3, 1, 1, 1, 1, 0, 1, b, st),
              FORGE_EINVAL);
    EXPECT_EQ(forge_int8_conv2d_forward(u16, i8, u16, u16, u16, 1, 16, 8, 8, 16, 0, 3, 1, 1, 1, 1, 1, 1, b, st),
              FORGE_EINVAL);
    EXPECT_EQ(forge_int8_conv2d_forward(u16, i8, u16, u16, u16, 1, 16, 8, 8, 16, 3, 3, -1, 1, 1, 1, 1, 1, b, st),
              FORGE_EINVAL);
    EXPECT_EQ(forge_int8_conv2d_forward(u16, i8, u16, u16, u16, 1, 16, INT_MAX, INT_MAX, 16, 3, 3, 1, 1, 1, 1, 1, 1,
                                        b, st),
              FORGE_EINVAL);
    EXPECT_EQ(forge_int8_conv2d_forward(u16, i8, u16, u16, u16, 1, 16, 2, 2, 16, 5, 5, 0, 0, 1, 1, 1, 1, b, st),
              FORGE_OK);   // empty output (kernel larger than the padded input)
    EXPECT_ERR(forge_int8_conv2d_forward(u16, i8, u16, u16, u16, 1, 16, 8, 8, 16, 3, 3, 1, 1, 1, 1, 1, 1, b, st));
    EXPECT_ERR(forge_int8_conv2d_forward(u16, i8, u16, u16, u16, 2, 3, 9, 7, 5, 3, 3, 1, 1, 2, 2, 1, 1, b, st));

    EXPECT_EQ(forge_int8_conv2d_nhwc_s32(nullptr, nullptr, nullptr, 0, 8, 8, 16, 16, 3, 3, 1, 1, 1, 1, 1, 1, st),
              FORGE_OK);
    EXPECT_EQ(forge_int8_conv2d_nhwc_s32(i8, i8, nullptr, 1, 8, 8, 16, 16, 3, 3, 1, 1, 1, 1, 1, 1, st), FORGE_EINVAL);
    EXPECT_EQ(forge_int8_conv2d_nhwc_s32(i8, i8, i32, 1, 8, 8, 16, 16, 3, 3, 1, 1, 0, 1, 1, 1, st), FORGE_EINVAL);
    EXPECT_EQ(forge_int8_conv2d_nhwc_s32(i8, i8, i32, 1, 8, 8, 16, 16, 3, 3, 1, 1, 1, 1, 1, -1, st), FORGE_EINVAL);
    EXPECT_EQ(forge_int8_conv2d_nhwc_s32(i8, i8, i32, 1, INT_MAX, INT_MAX, 16, 16, 3, 3, 1, 1, 1, 1, 1, 1, st),
              FORGE_EINVAL);
    EXPECT_ERR(forge_int8_conv2d_nhwc_s32(i8, i8, i32, 1, 8, 8, 16, 16, 3, 3, 1, 1, 1, 1, 1, 1, st));
    EXPECT_EQ(forge_int8_conv2d_nhwc_dequant(i8, i8, nullptr, u16, u16, u16, 1, 8, 8, 16, 16, 3, 3, 1, 1, 1, 1, 1, 1,
                                             st),
              FORGE_EINVAL);
    EXPECT_ERR(forge_int8_conv2d_nhwc_dequant(i8, i8, f32, u16, u16, u16, 1, 8, 8, 16, 16, 3, 3, 1, 1, 1, 1, 1, 1, st));

    EXPECT_EQ(forge_int8_conv_transpose2d_k2s2_forward(nullptr, nullptr, nullptr, nullptr, nullptr, 0, 16, 8, 8, 16,
                                                       nullptr, st),
              FORGE_OK);
    EXPECT_EQ(forge_int8_conv_transpose2d_k2s2_forward(u16, i8, u16, u16, u16, 1, 16, 8, 8, 16, nullptr, st),
              FORGE_EINVAL);
    EXPECT_EQ(forge_int8_conv_transpose2d_k2s2_forward(u16, i8, u16, u16, u16, 1, 16, INT_MAX, INT_MAX, 16, b, st),
              FORGE_EINVAL);
    EXPECT_ERR(forge_int8_conv_transpose2d_k2s2_forward(u16, i8, u16, u16, u16, 1, 16, 8, 8, 16, b, st));

    EXPECT_EQ(forge_int8_depthwise_conv2d_forward(nullptr, nullptr, nullptr, nullptr, nullptr, 0, 16, 8, 8, 3, 3, 1, 1,
                                                  1, 1, 1, 1, st),
              FORGE_OK);
    EXPECT_EQ(forge_int8_depthwise_conv2d_forward(u16, nullptr, u16, u16, u16, 1, 16, 8, 8, 3, 3, 1, 1, 1, 1, 1, 1, st),
              FORGE_EINVAL);
    EXPECT_EQ(forge_int8_depthwise_conv2d_forward(u16, i8, u16, u16, u16, 1, 16, 8, 8, 3, 3, 1, 1, 0, 1, 1, 1, st),
              FORGE_EINVAL);
    EXPECT_EQ(forge_int8_depthwise_conv2d_forward(u16, i8, u16, u16, u16, 1, 16, 8, 8, 3, 3, 1, 1, 1, 1, 1, 0, st),
              FORGE_EINVAL);
    EXPECT_EQ(forge_int8_depthwise_conv2d_forward(u16, i8, u16, u16, u16, 1, 16, INT_MAX, INT_MAX, 3, 3, 1, 1, 1, 1, 1,
                                                  1, st),
              FORGE_EINVAL);
    EXPECT_ERR(forge_int8_depthwise_conv2d_forward(u16, i8, u16, u16, u16, 1, 16, 8, 8, 3, 3, 1, 1, 1, 1, 1, 1, st));

    if (g_fail) return 1;
    std::printf("abi argument checks: all expectations hold\n");
    return 0;
}
