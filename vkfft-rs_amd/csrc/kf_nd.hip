// Role variants of the N-D axis shapes (C3: 4096 x 4096 f32, C4: 512^3 f64)
// that differ only in their nontemporal choice. Within a chunk, the first
// pass streams the caller's input (nontemporal loads) and leaves its output
// cached for the next pass; middle passes keep both sides cached; the last
// pass streams the result out (nontemporal stores).
#include "fft_kernels_impl.hpp"

namespace vkfx {

static const FixedKernel kTable[] = {
    // 4096-point rows, first pass of a chunk
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, float, 0, -1, 4096, 256, 1, 4, 4352, false, true, false, 16, 16, 16),
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, float, 0, 1, 4096, 256, 1, 4, 4352, false, true, false, 16, 16, 16),
    // split 4096 column axis: the 64-point column pass in the middle, the
    // 64-point row-of-columns pass last
    VKFX_FIXED_NT(KK_FS_A, IoFsA, float, 0, -1, 64, 8, 32, 30, 65, true, false, false, 8, 8),
    VKFX_FIXED_NT(KK_FS_A, IoFsA, float, 0, 1, 64, 8, 32, 30, 65, true, false, false, 8, 8),
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, float, 0, -1, 64, 8, 32, 30, 65, true, false, true, 8, 8),
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, float, 0, 1, 64, 8, 32, 30, 65, true, false, true, 8, 8),
    // f64 512: rows first, columns in the middle or last
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, double, 1, -1, 512, 64, 2, 3, 576, false, true, false, 8, 8, 8),
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, double, 1, 1, 512, 64, 2, 3, 576, false, true, false, 8, 8, 8),
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, double, 1, -1, 512, 64, 16, 30, 513, true, false, false, 8, 8, 8),
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, double, 1, 1, 512, 64, 16, 30, 513, true, false, false, 8, 8, 8),
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, double, 1, -1, 512, 64, 16, 30, 513, true, false, true, 8, 8, 8),
    VKFX_FIXED_NT(KK_PLAIN, IoPlain, double, 1, 1, 512, 64, 16, 30, 513, true, false, true, 8, 8, 8),
};

const FixedKernel* fixed_table_nd(int* count) {
    *count = (int)(sizeof(kTable) / sizeof(kTable[0]));
    return kTable;
}

}  // namespace vkfx
