// Fixed-shape C2C kernels for the contiguous and strided axes of the
// benchmark configurations (1024 and 4096 f32, 512 f64).
#include "fft_kernels_impl.hpp"

namespace vkfx {

static const FixedKernel kTable[] = {
    // 1-D rows of 1024 (C1): two waves per line, 8 elements per thread in the
    // radix-8 stages (16 in the radix-16 load stage), product-tree twiddles
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, float, 0, -1, 1024, 128, 1, 4, 1088, false, true, true, 16, 8, 8),
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, float, 0, 1, 1024, 128, 1, 4, 1088, false, true, true, 16, 8, 8),
    // per-stage twiddle tables and pads (VKFX_FIXED_PICK=1): half the rounding
    // error, 7% slower on two boxes (26.1 against 28.0 us)
    VKFX_FIXED_TS(KK_PLAIN, IoPlain, float, 0, -1, 1024, 128, 1, 4, 1088, false, 0, true, true, 16, 8, 8),
    VKFX_FIXED_TS(KK_PLAIN, IoPlain, float, 0, 1, 1024, 128, 1, 4, 1088, false, 0, true, true, 16, 8, 8),
    // one wave per line (VKFX_FIXED_PICK=2)
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, float, 0, -1, 1024, 64, 1, 5, 1056, false, true, true, 16, 16, 4),
    // the previous padding (one slot per 32; VKFX_FIXED_PICK=3)
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, float, 0, -1, 1024, 128, 1, 5, 1056, false, true, true, 16, 8, 8),
    // rows of 4096 (C3 axis 1; per-stage twiddle tables measured 6% slower here: 15 table loads per
    // radix-16 butterfly against the product tree's 14 multiplications)
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, float, 0, -1, 4096, 256, 1, 4, 4352, false, true, true, 16, 16, 16),
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, float, 0, 1, 4096, 256, 1, 4, 4352, false, true, true, 16, 16, 16),
    // columns of 4096 (C3 axis 0): 4 adjacent columns per block
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, float, 0, -1, 4096, 128, 4, 4, 4356, true, true, true, 16, 16, 16),
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, float, 0, 1, 4096, 128, 4, 4, 4356, true, true, true, 16, 16, 16),
    // f64 512 rows and columns (C4)
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, double, 1, -1, 512, 64, 2, 3, 576, false, true, true, 8, 8, 8),
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, double, 1, 1, 512, 64, 2, 3, 576, false, true, true, 8, 8, 8),
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, double, 1, -1, 512, 64, 16, 30, 513, true, true, true, 8, 8, 8),
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, double, 1, 1, 512, 64, 16, 30, 513, true, true, true, 8, 8, 8),
    // 64-point column passes of a split strided axis (4096 = 64 x 64): 32
    // adjacent columns per block, 256-byte row segments
    VKFX_FIXED_NT(KK_FS_A, IoFsA, float, 0, -1, 64, 8, 32, 30, 65, true, true, true, 8, 8),
    VKFX_FIXED_NT(KK_FS_A, IoFsA, float, 0, 1, 64, 8, 32, 30, 65, true, true, true, 8, 8),
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, float, 0, -1, 64, 8, 32, 30, 65, true, true, true, 8, 8),
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, float, 0, 1, 64, 8, 32, 30, 65, true, true, true, 8, 8),
};

const FixedKernel* fixed_table_plain(int* count) {
    *count = (int)(sizeof(kTable) / sizeof(kTable[0]));
    return kTable;
}

}  // namespace vkfx
