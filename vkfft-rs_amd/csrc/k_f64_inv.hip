// Kernel instantiations for one precision and first-FFT direction; split so
// the four variants compile in parallel.
#include "fft_kernels_impl.hpp"

namespace vkfx {
KernelFn pick_f64_inv(KernelKind kind, bool wide, int direct, int edge, bool rad) {
    return pick<double, 1>(kind, wide, direct, edge, rad);
}
}  // namespace vkfx
