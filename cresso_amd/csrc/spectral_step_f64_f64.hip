// Spectral step instantiated for double params and double grads (one translation
// unit per dtype pair, so that the pairs compile in parallel).
#include "spectral_kernels.hpp"

namespace cresso {
int32_t spectral_run_f64_f64(const cresso_spectral_plan& P, const cresso_spectral_desc* hd, int count,
                            const cresso_spectral_desc* dv, size_t ls, void* ws, const cresso_hyper& h, hipStream_t s) {
    return spectral_run<double, double>(P, hd, count, dv, ls, ws, h, s);
}
}  // namespace cresso
