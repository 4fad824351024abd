// Fixed-shape kernels of the two-upload real transforms (C2: N = 2^20, half
// size M = 2^19). Every block is one 1024-thread workgroup holding 128-148 KiB
// of lines in LDS, so each HBM access of a strided side moves 128-byte row
// segments (16 f32 complex columns, or 16 rows beside their 16 mirrors).
#include "fft_kernels_impl.hpp"

namespace vkfx {

static const FixedKernel kTable[] = {
    // R2C, M = 1024 x 512: 16 columns of 1024 per block, then 16 rows of 512
    // beside their 16 mirror rows (postprocess fused); the planner takes the
    // 512 x 1024 pair below when both are registered, these serve the C2C
    // four-step and VKFX_FIXED_PICK comparisons
    VKFX_FIXED_NT(KK_FS_A, IoFsA, float, 0, -1, 1024, 64, 16, 30, 1025, true, false, false, 16, 16, 4),
    VKFX_FIXED_NT(KK_FS_B_R2C, IoFsBR2C, float, 0, -1, 512, 32, 32, 4, 543, false, false, false, 8, 8, 8),
    // R2C, M = 512 x 1024: 32 columns of 512 per block (256-byte row
    // segments), then 8 rows of 1024 beside their 8 mirror rows
    VKFX_SHAPE(KK_FS_A, IoFsA, float, 0, -1, 512, 32, 32, 3, 577, true, false, false, 8, 8, 8),
    VKFX_SHAPE(KK_FS_B_R2C, IoFsBR2C, float, 0, -1, 1024, 64, 16, 4, 1089, false, false, false, 16, 16, 4),
    // C2R, M = 512 x 1024: 16 columns of 512 beside their 16 mirror columns
    // (preprocess fused), then 16 rows of 1024
    VKFX_FIXED_NT(KK_FS_A_C2R, IoFsAC2RDirect, float, 0, 1, 512, 32, 32, 3, 577, true, false, false, 8, 8, 8),
    VKFX_FIXED_NT(KK_FS_A_C2R, IoFsAC2R, float, 0, 1, 512, 32, 32, 3, 577, true, false, false, 8, 8, 8),
    VKFX_FIXED_NT(KK_FS_B, IoFsB, float, 0, 1, 1024, 64, 16, 4, 1089, false, false, false, 16, 16, 4),
    // row pass of the C2C four-step of 2^20 = 1024 x 1024 (its column pass is the first entry)
    VKFX_FIXED_NT(KK_FS_B, IoFsB, float, 0, -1, 1024, 64, 16, 4, 1089, false, false, false, 16, 16, 4),
    // earlier 512-thread shapes (VKFX_FIXED_PICK=1)
    VKFX_FIXED_NT(KK_FS_A, IoFsA, float, 0, -1, 1024, 64, 8, 4, 1092, true, false, false, 16, 16, 4),
    VKFX_FIXED_NT(KK_FS_B_R2C, IoFsBR2C, float, 0, -1, 512, 32, 16, 3, 578, false, false, false, 8, 8, 8),
    // the previous LDS paddings (VKFX_FIXED_PICK=2)
    VKFX_FIXED_NT(KK_FS_A, IoFsA, float, 0, -1, 1024, 64, 16, 4, 1090, true, false, false, 16, 16, 4),
    VKFX_FIXED_NT(KK_FS_B_R2C, IoFsBR2C, float, 0, -1, 512, 32, 32, 3, 577, false, false, false, 8, 8, 8),
    VKFX_FIXED_NT(KK_FS_B, IoFsB, float, 0, 1, 1024, 64, 16, 5, 1058, false, false, false, 16, 16, 4),
};

const FixedKernel* fixed_table_real(int* count) {
    *count = (int)(sizeof(kTable) / sizeof(kTable[0]));
    return kTable;
}

}  // namespace vkfx
