// Fixed-shape passes of the mixed-storage two-upload C2C (IoFsAEdge reads the
// half-precision input, IoFsBEdge writes the half-precision output) for the
// factors 256 ... 2048 of the four-step splits of 2^16 ... 2^22, with the
// threads, lines per block, radices and LDS strides of the four-step pass of
// the same length; nontemporal on the caller's side as the plain passes'
// roles are.
#include "fft_kernels_impl.hpp"

namespace vkfx {

#define VKFX_FS_EDGE_A(T, PREC, S, N, TT, G, PS, LS, ...) \
    VKFX_FIXED_NT(KK_FS_A_EDGE, IoFsAEdge, T, PREC, S, N, TT, G, PS, LS, true, true, false, __VA_ARGS__)
#define VKFX_FS_EDGE_B(T, PREC, S, N, TT, G, PS, LS, ...) \
    VKFX_FIXED_NT(KK_FS_B_EDGE, IoFsBEdge, T, PREC, S, N, TT, G, PS, LS, false, false, true, __VA_ARGS__)

// the shape of each (precision, direction, length) is the first registered
// KK_FS_A / KK_FS_B shape of that key (the plain pass the planner picks)
static const FixedKernel kTable[] = {
    VKFX_FS_EDGE_A(float, 0, -1, 256, 16, 32, 30, 257, 16, 16),
    VKFX_FS_EDGE_A(float, 0, 1, 256, 16, 32, 30, 257, 16, 16),
    VKFX_FS_EDGE_A(float, 0, -1, 512, 32, 32, 3, 577, 8, 8, 8),
    VKFX_FS_EDGE_A(float, 0, 1, 512, 64, 16, 30, 513, 8, 8, 8),
    VKFX_FS_EDGE_A(float, 0, -1, 1024, 64, 16, 30, 1025, 16, 16, 4),
    VKFX_FS_EDGE_A(float, 0, 1, 1024, 64, 16, 30, 1025, 16, 8, 8),
    VKFX_FS_EDGE_A(float, 0, -1, 2048, 128, 8, 30, 2049, 16, 16, 8),
    VKFX_FS_EDGE_A(float, 0, 1, 2048, 128, 8, 30, 2049, 16, 16, 8),
    VKFX_FS_EDGE_B(float, 0, -1, 256, 16, 16, 4, 273, 16, 16),
    VKFX_FS_EDGE_B(float, 0, 1, 256, 16, 16, 4, 273, 16, 16),
    VKFX_FS_EDGE_B(float, 0, -1, 512, 64, 16, 4, 545, 8, 8, 8),
    VKFX_FS_EDGE_B(float, 0, 1, 512, 64, 16, 4, 545, 8, 8, 8),
    VKFX_FS_EDGE_B(float, 0, -1, 1024, 64, 16, 4, 1089, 16, 16, 4),
    VKFX_FS_EDGE_B(float, 0, 1, 1024, 64, 16, 4, 1089, 16, 16, 4),
    VKFX_FS_EDGE_B(float, 0, -1, 2048, 128, 8, 4, 2177, 16, 16, 8),
    VKFX_FS_EDGE_B(float, 0, 1, 2048, 128, 8, 4, 2177, 16, 16, 8),
    VKFX_FS_EDGE_A(double, 1, -1, 256, 16, 32, 30, 257, 16, 16),
    VKFX_FS_EDGE_A(double, 1, 1, 256, 16, 32, 30, 257, 16, 16),
    VKFX_FS_EDGE_A(double, 1, -1, 512, 64, 16, 30, 513, 8, 8, 8),
    VKFX_FS_EDGE_A(double, 1, 1, 512, 64, 16, 30, 513, 8, 8, 8),
    VKFX_FS_EDGE_A(double, 1, -1, 1024, 64, 8, 30, 1025, 16, 8, 8),
    VKFX_FS_EDGE_A(double, 1, 1, 1024, 64, 8, 30, 1025, 16, 8, 8),
    VKFX_FS_EDGE_A(double, 1, -1, 2048, 128, 4, 30, 2049, 16, 16, 8),
    VKFX_FS_EDGE_A(double, 1, 1, 2048, 128, 4, 30, 2049, 16, 16, 8),
    VKFX_FS_EDGE_B(double, 1, -1, 256, 16, 16, 3, 289, 16, 16),
    VKFX_FS_EDGE_B(double, 1, 1, 256, 16, 16, 3, 289, 16, 16),
    VKFX_FS_EDGE_B(double, 1, -1, 512, 64, 16, 3, 577, 8, 8, 8),
    VKFX_FS_EDGE_B(double, 1, 1, 512, 64, 16, 3, 577, 8, 8, 8),
    VKFX_FS_EDGE_B(double, 1, -1, 1024, 64, 8, 3, 1153, 16, 8, 8),
    VKFX_FS_EDGE_B(double, 1, 1, 1024, 64, 8, 3, 1153, 16, 8, 8),
    VKFX_FS_EDGE_B(double, 1, -1, 2048, 128, 4, 3, 2305, 16, 16, 8),
    VKFX_FS_EDGE_B(double, 1, 1, 2048, 128, 4, 3, 2305, 16, 16, 8),
};

const FixedKernel* fixed_table_fs_edge(int* count) {
    *count = (int)(sizeof(kTable) / sizeof(kTable[0]));
    return kTable;
}

}  // namespace vkfx
