// Fixed-shape kernels of the two-upload real transforms (C2: N = 2^20, half
// size 2^19 = 1024 x 512).
#include "fft_kernels_impl.hpp"

namespace vkfx {

static const FixedKernel kTable[] = {
    // R2C: column pass over the packed half-size input, then mirror-row pass
    VKFX_FIXED_NT(KK_FS_A, IoFsA, float, 0, -1, 1024, 64, 8, 4, 1092, true, false, false, 16, 16, 4),
    VKFX_FIXED_NT(KK_FS_B_R2C, IoFsBR2C, float, 0, -1, 512, 32, 16, 3, 578, false, false, false, 8, 8, 8),
    // C2R: preprocess fused into the column pass, then the row pass
    VKFX_FIXED_NT(KK_FS_A_C2R, IoFsAC2R, float, 0, 1, 1024, 64, 8, 4, 1092, true, false, false, 16, 16, 4),
    VKFX_FIXED_NT(KK_FS_B, IoFsB, float, 0, 1, 512, 32, 16, 3, 578, false, false, false, 8, 8, 8),
    // row pass of the C2C four-step of 2^20 = 1024 x 1024 (its column pass is the entry above)
    VKFX_FIXED_NT(KK_FS_B, IoFsB, float, 0, -1, 1024, 64, 4, 5, 1064, false, false, false, 16, 16, 4),
};

const FixedKernel* fixed_table_real(int* count) {
    *count = (int)(sizeof(kTable) / sizeof(kTable[0]));
    return kTable;
}

}  // namespace vkfx
