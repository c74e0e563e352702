// Q4 GEMV kernel variants: epilogue residual, gated head RMSNorm prologue.
#include "q4_gemv_launch.hpp"

namespace prg {
template int launch_m<kEpiResidual, kNormGated>(hipStream_t, const GemvParams&, int, int, int, size_t);
}  // namespace prg
