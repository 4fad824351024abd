// Fixed-shape Bluestein kernels: M = 8232 (N = 4099) in one kernel of 686
// threads per line, M = 131220 = 405 x 324 (N = 65537) in three passes.
#include "fft_kernels_impl.hpp"

namespace vkfx {

static const FixedKernel kTable[] = {
    // M = 8232: in place with per-stage twiddle tables and pads, at most 80
    // VGPRs (74, no spill) so two 74 KiB blocks share a CU; then the ping-pong form (one block per
    // CU, one barrier per stage) and the in-place form with product-tree
    // twiddles and one uniform pad (VKFX_FIXED_PICK_K12=1, 2). Without the
    // spill, 588 threads per line (88 VGPRs, radix-7 stages in two exact
    // rounds) ran 260 us and 392 threads (123 VGPRs) 223 us, against 192 us
    VKFX_FIXED_TS(KK_BLUE_1, IoBlue1, float, 0, -1, 8232, 686, 1, 3, 9261, false, 6, true, true, 8, 3, 7, 7, 7),
    VKFX_FIXED_PPTS(KK_BLUE_1, IoBlue1, float, 0, -1, 8232, 686, 1, 3, 9261, false, true, true, 8, 3, 7, 7, 7),
    VKFX_FIXED_NT(KK_BLUE_1, IoBlue1, float, 0, -1, 8232, 686, 1, 5, 8489, false, true, true, 8, 3, 7, 7, 7),
    // the first M = 8232 shape with the 1-D boundary work inside (storage
    // conversion and zero intervals)
    VKFX_FIXED_TS(KK_BLUE_1_EDGE, IoBlue1Edge, float, 0, -1, 8232, 686, 1, 3, 9261, false, 6, true, true, 8, 3, 7, 7, 7),
    // M = 131220: product-tree twiddles (per-stage tables measured 4% slower;
    // on the row pass 10-20% slower). Column passes of 405 with 45 threads
    // per column (one radix-9 butterfly each: 1.3% over 27 threads, the second
    // variant; 8 columns per block, 64-byte row segments, ran 5-14% slower;
    // 15 threads per column with radices 27 and 15, two LDS exchanges
    // instead of three and 30% fewer instructions per element but 101-117
    // VGPRs, took C5b from 5.04-5.07 to 5.20-5.24 ms, its inverse column pass
    // from 58 to 72 us). The 324-point row pass: 18 threads per row, two
    // radix-18 stages (nine-by-two composite butterflies: 121 instead of 156
    // VALU instructions per element, 7 instead of 11 barriers, 94 VGPRs),
    // 7 rows per block, C5b 5.06-5.08 against 5.16 ms for the second variant
    // (36 threads per row, radix 4, 9, 9, 7 rows: 252 threads fill four
    // waves; 8 rows, 3, 5 and 14 rows, an odd line stride, 27 threads per row
    // and the radix orders 9-9-4 and 9-4-9 ran slower; 14 rows of 18 threads
    // measured the same as 7)
    VKFX_FIXED_NT(KK_FS_A_BLUE, IoFsABlue, float, 0, -1, 405, 45, 16, 30, 405, true, true, false, 9, 9, 5),
    VKFX_FIXED_NT(KK_FS_C_BLUE, IoFsCBlue, float, 0, 1, 405, 45, 16, 30, 405, true, false, true, 9, 9, 5),
    VKFX_FIXED_NT(KK_FS_A_BLUE, IoFsABlue, float, 0, -1, 405, 27, 16, 30, 407, true, true, false, 9, 9, 5),
    VKFX_FIXED_NT(KK_FS_C_BLUE, IoFsCBlue, float, 0, 1, 405, 27, 16, 30, 407, true, false, true, 9, 9, 5),
    VKFX_FIXED_NT(KK_BLUE_B, IoBlueB, float, 0, -1, 324, 18, 7, 30, 324, false, false, false, 18, 18),
    VKFX_FIXED_NT(KK_BLUE_B, IoBlueB, float, 0, -1, 324, 36, 7, 30, 324, false, false, false, 4, 9, 9),
};

const FixedKernel* fixed_table_blue(int* count) {
    *count = (int)(sizeof(kTable) / sizeof(kTable[0]));
    return kTable;
}

}  // namespace vkfx
