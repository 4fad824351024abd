// Fixed shapes of the one-upload even-length real transforms, f32: the
// half-size packed FFT of R2C (postprocess fused into the staged store) and of
// C2R (preprocess fused into the direct loads) for half lengths M that have a
// fixed C2C row shape (powers of two and the 3*2^k / 5*2^k families), with the
// same radices, threads, lines per block and LDS strides as those rows. R2C is
// registered for the caller's input with or without the caller's output, C2R
// for the caller's output with or without the caller's input.
#include "fft_kernels_impl.hpp"

namespace vkfx {

static const FixedKernel kTable[] = {
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 256, 16, 16, 4, 271, false, true, true, 16, 16),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 256, 16, 16, 4, 271, false, true, false, 16, 16),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 256, 16, 16, 4, 271, false, true, true, 16, 16),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 256, 16, 16, 4, 271, false, false, true, 16, 16),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 512, 64, 4, 4, 543, false, true, true, 8, 8, 8),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 512, 64, 4, 4, 543, false, true, false, 8, 8, 8),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 512, 64, 4, 4, 543, false, true, true, 8, 8, 8),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 512, 64, 4, 4, 543, false, false, true, 8, 8, 8),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 1024, 128, 1, 4, 1088, false, true, true, 16, 8, 8),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 1024, 128, 1, 4, 1088, false, true, false, 16, 8, 8),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 1024, 128, 1, 4, 1088, false, true, true, 16, 8, 8),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 1024, 128, 1, 4, 1088, false, false, true, 16, 8, 8),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 2048, 256, 1, 4, 2175, false, true, true, 16, 16, 8),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 2048, 256, 1, 4, 2175, false, true, false, 16, 16, 8),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 2048, 256, 1, 4, 2175, false, true, true, 16, 16, 8),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 2048, 256, 1, 4, 2175, false, false, true, 16, 16, 8),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 4096, 256, 1, 4, 4352, false, true, true, 16, 16, 16),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 4096, 256, 1, 4, 4352, false, true, false, 16, 16, 16),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 4096, 256, 1, 4, 4352, false, true, true, 16, 16, 16),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 4096, 256, 1, 4, 4352, false, false, true, 16, 16, 16),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 8192, 512, 1, 4, 8703, false, true, true, 16, 16, 8, 4),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 8192, 512, 1, 4, 8703, false, true, false, 16, 16, 8, 4),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 8192, 512, 1, 4, 8703, false, true, true, 16, 16, 8, 4),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 8192, 512, 1, 4, 8703, false, false, true, 16, 16, 8, 4),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 384, 24, 10, 4, 409, false, true, true, 16, 8, 3),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 384, 24, 10, 4, 409, false, true, false, 16, 8, 3),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 384, 24, 10, 4, 409, false, true, true, 16, 8, 3),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 384, 24, 10, 4, 409, false, false, true, 16, 8, 3),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 768, 48, 5, 4, 815, false, true, true, 16, 16, 3),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 768, 48, 5, 4, 815, false, true, false, 16, 16, 3),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 768, 48, 5, 4, 815, false, true, true, 16, 16, 3),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 768, 48, 5, 4, 815, false, false, true, 16, 16, 3),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 1536, 96, 2, 4, 1631, false, true, true, 16, 16, 6),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 1536, 96, 2, 4, 1631, false, true, false, 16, 16, 6),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 1536, 96, 2, 4, 1631, false, true, true, 16, 16, 6),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 1536, 96, 2, 4, 1631, false, false, true, 16, 16, 6),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 3072, 192, 1, 4, 3263, false, true, true, 16, 16, 12),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 3072, 192, 1, 4, 3263, false, true, false, 16, 16, 12),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 3072, 192, 1, 4, 3263, false, true, true, 16, 16, 12),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 3072, 192, 1, 4, 3263, false, false, true, 16, 16, 12),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 6144, 384, 1, 4, 6527, false, true, true, 16, 16, 8, 3),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 6144, 384, 1, 4, 6527, false, true, false, 16, 16, 8, 3),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 6144, 384, 1, 4, 6527, false, true, true, 16, 16, 8, 3),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 6144, 384, 1, 4, 6527, false, false, true, 16, 16, 8, 3),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 320, 40, 6, 3, 360, false, true, true, 8, 8, 5),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 320, 40, 6, 3, 360, false, true, false, 8, 8, 5),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 320, 40, 6, 3, 360, false, true, true, 8, 8, 5),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 320, 40, 6, 3, 360, false, false, true, 8, 8, 5),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 640, 40, 6, 4, 680, false, true, true, 16, 8, 5),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 640, 40, 6, 4, 680, false, true, false, 16, 8, 5),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 640, 40, 6, 4, 680, false, true, true, 16, 8, 5),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 640, 40, 6, 4, 680, false, false, true, 16, 8, 5),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 1280, 80, 3, 4, 1359, false, true, true, 16, 16, 5),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 1280, 80, 3, 4, 1359, false, true, false, 16, 16, 5),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 1280, 80, 3, 4, 1359, false, true, true, 16, 16, 5),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 1280, 80, 3, 4, 1359, false, false, true, 16, 16, 5),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 2560, 160, 1, 4, 2719, false, true, true, 16, 16, 10),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 2560, 160, 1, 4, 2719, false, true, false, 16, 16, 10),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 2560, 160, 1, 4, 2719, false, true, true, 16, 16, 10),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 2560, 160, 1, 4, 2719, false, false, true, 16, 16, 10),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 5120, 320, 1, 4, 5439, false, true, true, 16, 16, 4, 5),
    VKFX_SHAPE(KK_R2C_HALF, IoR2CHalf, float, 0, -1, 5120, 320, 1, 4, 5439, false, true, false, 16, 16, 4, 5),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 5120, 320, 1, 4, 5439, false, true, true, 16, 16, 4, 5),
    VKFX_SHAPE(KK_C2R_HALF, IoC2RHalf, float, 0, 1, 5120, 320, 1, 4, 5439, false, false, true, 16, 16, 4, 5),
};

const FixedKernel* fixed_table_real_rows_f32(int* count) {
    *count = (int)(sizeof(kTable) / sizeof(kTable[0]));
    return kTable;
}

}  // namespace vkfx
