// Q4 GEMV kernel variants: epilogue plain, fused RMSNorm prologue.
#include "q4_gemv_launch.hpp"

namespace prg {
template int launch_m<kEpiPlain, kNormRms>(hipStream_t, const GemvParams&, int, int, int, size_t);
}  // namespace prg
