// Fixed shapes of the power-of-two lengths outside the benchmark
// configurations, f64: rows of one upload (1-D batches and the contiguous
// axis of N-D transforms), strided columns up to the length that stays one
// upload per axis, and the first pass of split strided axes. Each shape is
// registered for both directions and for the two nontemporal roles its pass
// can take (rows: the caller's input, with or without the caller's output;
// columns: cached input, with or without the caller's output). LDS strides
// minimise bank conflicts under the 32-bank model of 8-byte accesses (16 lanes
// served per cycle). Short rows, whose first or last Stockham stage would touch
// HBM in segments narrower than 128 bytes, stage both ends through LDS
// (IoPlainStaged).
#include "fft_kernels_impl.hpp"

namespace vkfx {

static const FixedKernel kTable[] = {
    VKFX_SHAPE(KK_PLAIN, IoPlainStaged, double, 1, -1, 8, 1, 64, 3, 9, false, true, true, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlainStaged, double, 1, -1, 8, 1, 64, 3, 9, false, true, false, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlainStaged, double, 1, 1, 8, 1, 64, 3, 9, false, true, true, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlainStaged, double, 1, 1, 8, 1, 64, 3, 9, false, true, false, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlainStaged, double, 1, -1, 16, 1, 64, 3, 17, false, true, true, 16),
    VKFX_SHAPE(KK_PLAIN, IoPlainStaged, double, 1, -1, 16, 1, 64, 3, 17, false, true, false, 16),
    VKFX_SHAPE(KK_PLAIN, IoPlainStaged, double, 1, 1, 16, 1, 64, 3, 17, false, true, true, 16),
    VKFX_SHAPE(KK_PLAIN, IoPlainStaged, double, 1, 1, 16, 1, 64, 3, 17, false, true, false, 16),
    VKFX_SHAPE(KK_PLAIN, IoPlainStaged, double, 1, -1, 32, 8, 32, 3, 35, false, true, true, 8, 4),
    VKFX_SHAPE(KK_PLAIN, IoPlainStaged, double, 1, -1, 32, 8, 32, 3, 35, false, true, false, 8, 4),
    VKFX_SHAPE(KK_PLAIN, IoPlainStaged, double, 1, 1, 32, 8, 32, 3, 35, false, true, true, 8, 4),
    VKFX_SHAPE(KK_PLAIN, IoPlainStaged, double, 1, 1, 32, 8, 32, 3, 35, false, true, false, 8, 4),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 64, 8, 32, 3, 71, false, true, true, 8, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 64, 8, 32, 3, 71, false, true, false, 8, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 64, 8, 32, 3, 71, false, true, true, 8, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 64, 8, 32, 3, 71, false, true, false, 8, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 128, 16, 16, 4, 135, false, true, true, 16, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 128, 16, 16, 4, 135, false, true, false, 16, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 128, 16, 16, 4, 135, false, true, true, 16, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 128, 16, 16, 4, 135, false, true, false, 16, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 256, 16, 16, 4, 271, false, true, true, 16, 16),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 256, 16, 16, 4, 271, false, true, false, 16, 16),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 256, 16, 16, 4, 271, false, true, true, 16, 16),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 256, 16, 16, 4, 271, false, true, false, 16, 16),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 1024, 128, 2, 4, 1087, false, true, true, 16, 8, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 1024, 128, 2, 4, 1087, false, true, false, 16, 8, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 1024, 128, 2, 4, 1087, false, true, true, 16, 8, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 1024, 128, 2, 4, 1087, false, true, false, 16, 8, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 2048, 256, 1, 4, 2175, false, true, true, 16, 16, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 2048, 256, 1, 4, 2175, false, true, false, 16, 16, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 2048, 256, 1, 4, 2175, false, true, true, 16, 16, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 2048, 256, 1, 4, 2175, false, true, false, 16, 16, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 4096, 256, 1, 4, 4351, false, true, true, 16, 16, 16),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 4096, 256, 1, 4, 4351, false, true, false, 16, 16, 16),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 4096, 256, 1, 4, 4351, false, true, true, 16, 16, 16),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 4096, 256, 1, 4, 4351, false, true, false, 16, 16, 16),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 8192, 512, 1, 4, 8703, false, true, true, 16, 16, 8, 4),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 8192, 512, 1, 4, 8703, false, true, false, 16, 16, 8, 4),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 8192, 512, 1, 4, 8703, false, true, true, 16, 16, 8, 4),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 8192, 512, 1, 4, 8703, false, true, false, 16, 16, 8, 4),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 8, 1, 64, 3, 8, true, false, false, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 8, 1, 64, 3, 8, true, false, true, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 8, 1, 64, 3, 8, true, false, false, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 8, 1, 64, 3, 8, true, false, true, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 16, 1, 64, 4, 16, true, false, false, 16),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 16, 1, 64, 4, 16, true, false, true, 16),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 16, 1, 64, 4, 16, true, false, false, 16),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 16, 1, 64, 4, 16, true, false, true, 16),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 32, 8, 32, 4, 33, true, false, false, 8, 4),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 32, 8, 32, 4, 33, true, false, true, 8, 4),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 32, 8, 32, 4, 33, true, false, false, 8, 4),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 32, 8, 32, 4, 33, true, false, true, 8, 4),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 64, 8, 32, 5, 65, true, false, false, 8, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 64, 8, 32, 5, 65, true, false, true, 8, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 64, 8, 32, 5, 65, true, false, false, 8, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 64, 8, 32, 5, 65, true, false, true, 8, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 128, 16, 16, 6, 129, true, false, false, 16, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 128, 16, 16, 6, 129, true, false, true, 16, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 128, 16, 16, 6, 129, true, false, false, 16, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 128, 16, 16, 6, 129, true, false, true, 16, 8),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 256, 16, 16, 30, 257, true, false, false, 16, 16),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, -1, 256, 16, 16, 30, 257, true, false, true, 16, 16),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 256, 16, 16, 30, 257, true, false, false, 16, 16),
    VKFX_SHAPE(KK_PLAIN, IoPlain, double, 1, 1, 256, 16, 16, 30, 257, true, false, true, 16, 16),
    VKFX_SHAPE(KK_FS_A, IoFsA, double, 1, -1, 32, 8, 32, 4, 33, true, false, false, 8, 4),
    VKFX_SHAPE(KK_FS_A, IoFsA, double, 1, 1, 32, 8, 32, 4, 33, true, false, false, 8, 4),
    VKFX_SHAPE(KK_FS_A, IoFsA, double, 1, -1, 64, 8, 32, 5, 65, true, false, false, 8, 8),
    VKFX_SHAPE(KK_FS_A, IoFsA, double, 1, 1, 64, 8, 32, 5, 65, true, false, false, 8, 8),
    VKFX_SHAPE(KK_FS_A, IoFsA, double, 1, -1, 128, 16, 16, 6, 129, true, false, false, 16, 8),
    VKFX_SHAPE(KK_FS_A, IoFsA, double, 1, 1, 128, 16, 16, 6, 129, true, false, false, 16, 8),
};

const FixedKernel* fixed_table_pow2_f64(int* count) {
    *count = (int)(sizeof(kTable) / sizeof(kTable[0]));
    return kTable;
}

}  // namespace vkfx
