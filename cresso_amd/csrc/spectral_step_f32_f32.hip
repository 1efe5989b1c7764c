// Spectral step instantiated for float params and float grads (one translation
// unit per dtype pair, so that the pairs compile in parallel).
#include "spectral_kernels.hpp"

namespace cresso {
int32_t spectral_run_f32_f32(const cresso_spectral_plan& P, const cresso_spectral_desc& d, void* ws,
                            const cresso_hyper& h, hipStream_t s) {
    return spectral_run<float, float>(P, d, ws, h, s);
}
}  // namespace cresso
