// Q4 GEMV kernel variants: epilogue residual.
#include "q4_gemv_launch.hpp"

namespace prg {
template int launch_m<kEpiResidual, kNormNone>(hipStream_t, const GemvParams&, int, int, int, size_t);
}  // namespace prg
