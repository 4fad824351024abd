// Fixed-shape Bluestein kernels: M = 8232 (N = 4099) in one kernel of 686
// threads per line, M = 131220 = 405 x 324 (N = 65537) in three passes.
#include "fft_kernels_impl.hpp"

namespace vkfx {

static const FixedKernel kTable[] = {
    // M = 8232: in place with per-stage twiddle tables and pads, 80 VGPRs so
    // two 74 KiB blocks share a CU; then the ping-pong form (one block per
    // CU, one barrier per stage) and the in-place form with product-tree
    // twiddles and one uniform pad (VKFX_FIXED_PICK_K12=1, 2)
    VKFX_FIXED_TS(KK_BLUE_1, IoBlue1, float, 0, -1, 8232, 686, 1, 3, 9261, false, 6, true, true, 8, 3, 7, 7, 7),
    VKFX_FIXED_PPTS(KK_BLUE_1, IoBlue1, float, 0, -1, 8232, 686, 1, 3, 9261, false, true, true, 8, 3, 7, 7, 7),
    VKFX_FIXED_NT(KK_BLUE_1, IoBlue1, float, 0, -1, 8232, 686, 1, 5, 8489, false, true, true, 8, 3, 7, 7, 7),
    // M = 131220: product-tree twiddles (per-stage tables measured 4% slower).
    // Column passes of 405 with 45 threads per column (one radix-9 butterfly
    // each: 1.3% over 27 threads, the second variant); the 324-point row pass
    // with 36 threads per row (radix 4, 9, 9: one radix-9 butterfly per thread,
    // three radix-4 rounds) and 8 rows per block, 6-7% over 27 threads per row
    // (the second variant) on two boxes; 16 rows per block, an LDS pad of one
    // per 16, radix orders 9-9-4 / 9-4-9 (fewer modelled LDS bank conflicts)
    // and 81 threads per row ran slower (5.50-6.86 ms against 5.41-5.47)
    VKFX_FIXED_NT(KK_FS_A_BLUE, IoFsABlue, float, 0, -1, 405, 45, 16, 30, 405, true, true, false, 9, 9, 5),
    VKFX_FIXED_NT(KK_FS_C_BLUE, IoFsCBlue, float, 0, 1, 405, 45, 16, 30, 405, true, false, true, 9, 9, 5),
    VKFX_FIXED_NT(KK_FS_A_BLUE, IoFsABlue, float, 0, -1, 405, 27, 16, 30, 407, true, true, false, 9, 9, 5),
    VKFX_FIXED_NT(KK_FS_C_BLUE, IoFsCBlue, float, 0, 1, 405, 27, 16, 30, 407, true, false, true, 9, 9, 5),
    VKFX_FIXED_NT(KK_BLUE_B, IoBlueB, float, 0, -1, 324, 36, 8, 30, 324, false, false, false, 4, 9, 9),
    VKFX_FIXED_NT(KK_BLUE_B, IoBlueB, float, 0, -1, 324, 27, 8, 30, 347, false, false, false, 4, 9, 9),
};

const FixedKernel* fixed_table_blue(int* count) {
    *count = (int)(sizeof(kTable) / sizeof(kTable[0]));
    return kTable;
}

}  // namespace vkfx
