// Fixed-shape Bluestein kernels (C5): N = 4099 with M = 8232 in one kernel
// (686 threads per line; VKFX_FIXED_PICK=1 selects 448),
// N = 65537 with M = 131220 = 405 x 324 in three passes.
#include "fft_kernels_impl.hpp"

namespace vkfx {

static const FixedKernel kTable[] = {
    VKFX_FIXED_NT(KK_BLUE_1, IoBlue1, float, 0, -1, 8232, 686, 1, 5, 8489, false, true, true, 8, 3, 7, 7, 7),
    VKFX_FIXED_NT(KK_BLUE_1, IoBlue1, float, 0, -1, 8232, 448, 1, 5, 8489, false, true, true, 8, 3, 7, 7, 7),
    VKFX_FIXED_NT(KK_FS_A_BLUE, IoFsABlue, float, 0, -1, 405, 27, 16, 30, 407, true, true, false, 9, 9, 5),
    VKFX_FIXED_NT(KK_BLUE_B, IoBlueB, float, 0, -1, 324, 27, 8, 30, 347, false, false, false, 4, 9, 9),
    VKFX_FIXED_NT(KK_FS_C_BLUE, IoFsCBlue, float, 0, 1, 405, 27, 16, 30, 407, true, false, true, 9, 9, 5),
};

const FixedKernel* fixed_table_blue(int* count) {
    *count = (int)(sizeof(kTable) / sizeof(kTable[0]));
    return kTable;
}

}  // namespace vkfx
