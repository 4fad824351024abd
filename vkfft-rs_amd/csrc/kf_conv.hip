// Fixed shapes of the convolution kernels. kTable: row passes of the
// two-upload convolution (IoConvB) for the row lengths N2 of the four-step
// splits of 2^16 ... 2^22, 10^5 and 10^6, with the threads per row, radices
// and LDS strides of the four-step row pass of the same length. Rows per
// block measured (fused convolution, ms): f32 512 8 rows 0.214 / 16 rows
// 0.224 (2^18 x 64), 1024 8 rows 0.257 / 16 rows 0.267 (2^20 x 16), 2048
// 8 rows 0.310 / 4 rows 0.331 (2^22 x 4); f64 512 8 rows 0.202 / 16 rows
// 0.220 (2^18 x 32), 1024 4 rows 0.222 / 8 rows 0.230 (2^20 x 8); f64 1000
// at 8 rows spills 64 bytes per lane (4 rows here).
#include "fft_kernels_impl.hpp"

namespace vkfx {

static const FixedKernel kTable[] = {
    VKFX_SHAPE(KK_CONV_B, IoConvB, float, 0, -1, 250, 25, 16, 4, 265, false, false, false, 10, 5, 5),
    VKFX_SHAPE(KK_CONV_B, IoConvB, float, 0, -1, 256, 16, 16, 4, 273, false, false, false, 16, 16),
    VKFX_SHAPE(KK_CONV_B, IoConvB, float, 0, -1, 512, 64, 8, 4, 545, false, false, false, 8, 8, 8),
    VKFX_SHAPE(KK_CONV_B, IoConvB, float, 0, -1, 1000, 100, 8, 4, 1063, false, false, false, 10, 10, 10),
    VKFX_SHAPE(KK_CONV_B, IoConvB, float, 0, -1, 1024, 64, 8, 4, 1089, false, false, false, 16, 16, 4),
    VKFX_SHAPE(KK_CONV_B, IoConvB, float, 0, -1, 2048, 128, 8, 4, 2177, false, false, false, 16, 16, 8),
    VKFX_SHAPE(KK_CONV_B, IoConvB, double, 1, -1, 250, 25, 16, 3, 281, false, false, false, 10, 5, 5),
    VKFX_SHAPE(KK_CONV_B, IoConvB, double, 1, -1, 256, 16, 16, 3, 289, false, false, false, 16, 16),
    VKFX_SHAPE(KK_CONV_B, IoConvB, double, 1, -1, 512, 64, 8, 3, 577, false, false, false, 8, 8, 8),
    VKFX_SHAPE(KK_CONV_B, IoConvB, double, 1, -1, 1000, 100, 4, 3, 1125, false, false, false, 10, 10, 10),
    VKFX_SHAPE(KK_CONV_B, IoConvB, double, 1, -1, 1024, 64, 4, 3, 1153, false, false, false, 16, 8, 8),
    VKFX_SHAPE(KK_CONV_B, IoConvB, double, 1, -1, 2048, 128, 4, 3, 2305, false, false, false, 16, 16, 8),
};

// One-upload convolutions (IoConv1F): rows of 1-D convolutions and axis-0
// columns of N-D ones, with the threads, lines per block, radices and LDS
// strides of the plain pass the planner picks for the same length and lane
// mapping.
static const FixedKernel kTable1[] = {
    VKFX_SHAPE(KK_CONV_1, IoConv1F, float, 0, -1, 256, 16, 16, 4, 271, false, true, true, 16, 16),
    VKFX_SHAPE(KK_CONV_1, IoConv1F, float, 0, -1, 512, 64, 4, 4, 543, false, true, true, 8, 8, 8),
    VKFX_SHAPE(KK_CONV_1, IoConv1F, float, 0, -1, 1024, 128, 1, 4, 1088, false, true, true, 16, 8, 8),
    VKFX_SHAPE(KK_CONV_1, IoConv1F, float, 0, -1, 2048, 256, 1, 4, 2175, false, true, true, 16, 16, 8),
    VKFX_SHAPE(KK_CONV_1, IoConv1F, float, 0, -1, 4096, 256, 1, 4, 4352, false, true, true, 16, 16, 16),
    VKFX_SHAPE(KK_CONV_1, IoConv1F, float, 0, -1, 8192, 512, 1, 4, 8703, false, true, true, 16, 16, 8, 4),
    VKFX_SHAPE(KK_CONV_1, IoConv1F, float, 0, -1, 64, 8, 32, 30, 65, true, true, true, 8, 8),
    VKFX_SHAPE(KK_CONV_1, IoConv1F, float, 0, -1, 128, 16, 16, 6, 129, true, true, true, 16, 8),
    VKFX_SHAPE(KK_CONV_1, IoConv1F, float, 0, -1, 256, 16, 16, 30, 257, true, true, true, 16, 16),
    VKFX_SHAPE(KK_CONV_1, IoConv1F, float, 0, -1, 512, 64, 16, 30, 513, true, true, true, 8, 8, 8),
    VKFX_SHAPE(KK_CONV_1, IoConv1F, double, 1, -1, 256, 16, 16, 4, 271, false, true, true, 16, 16),
    VKFX_SHAPE(KK_CONV_1, IoConv1F, double, 1, -1, 512, 64, 2, 3, 576, false, true, true, 8, 8, 8),
    VKFX_SHAPE(KK_CONV_1, IoConv1F, double, 1, -1, 1024, 128, 2, 4, 1087, false, true, true, 16, 8, 8),
    VKFX_SHAPE(KK_CONV_1, IoConv1F, double, 1, -1, 2048, 256, 1, 4, 2175, false, true, true, 16, 16, 8),
    VKFX_SHAPE(KK_CONV_1, IoConv1F, double, 1, -1, 4096, 256, 1, 4, 4351, false, true, true, 16, 16, 16),
    VKFX_SHAPE(KK_CONV_1, IoConv1F, double, 1, -1, 64, 8, 32, 5, 65, true, true, true, 8, 8),
    VKFX_SHAPE(KK_CONV_1, IoConv1F, double, 1, -1, 128, 16, 16, 6, 129, true, true, true, 16, 8),
    VKFX_SHAPE(KK_CONV_1, IoConv1F, double, 1, -1, 256, 16, 16, 30, 257, true, true, true, 16, 16),
    VKFX_SHAPE(KK_CONV_1, IoConv1F, double, 1, -1, 512, 64, 16, 30, 513, true, true, true, 8, 8, 8),
};

const FixedKernel* fixed_table_conv1(int* count) {
    *count = (int)(sizeof(kTable1) / sizeof(kTable1[0]));
    return kTable1;
}

const FixedKernel* fixed_table_conv(int* count) {
    *count = (int)(sizeof(kTable) / sizeof(kTable[0]));
    return kTable;
}

}  // namespace vkfx
