// Register-exchange kernel (fft_wave.hpp): one wave per 1024-point f32 line,
// every exchange between passes in registers, no LDS. Registered after the
// LDS-staged two-wave shape of the same key, which measured 1-4% faster on
// C1 (N=1024, batch 8192); plans built with VKFX_REGISTER_EXCHANGE=1 take
// this one, and the tests run both.
#include "fft_wave.hpp"

namespace vkfx {

// G = 4 lines per 256-thread block, TT = 64 threads per line.
#define VKFX_WAVE1024(S, NTI, NTO)                                                                    \
    FixedKernel {                                                                                     \
        KK_PLAIN, 0, S, 1024, 64, 4, 0, 0, false, NTI, NTO, 0, {16, 4, 16},                             \
            (KernelFn)(k_wave1024<S, NTI, NTO>), FT_WAVE1024                                            \
    }

static const FixedKernel kTable[] = {
    VKFX_WAVE1024(-1, true, true),  VKFX_WAVE1024(1, true, true),   VKFX_WAVE1024(-1, false, false),
    VKFX_WAVE1024(1, false, false), VKFX_WAVE1024(-1, true, false), VKFX_WAVE1024(1, true, false),
    VKFX_WAVE1024(-1, false, true), VKFX_WAVE1024(1, false, true),
};

const FixedKernel* fixed_table_wave(int* count) {
    *count = (int)(sizeof(kTable) / sizeof(kTable[0]));
    return kTable;
}

}  // namespace vkfx
