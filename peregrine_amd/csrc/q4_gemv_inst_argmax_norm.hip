// Q4 GEMV kernel variants: epilogue argmax, fused RMSNorm prologue.
#include "q4_gemv_launch.hpp"

namespace prg {
template int launch_m<kEpiArgmax, kNormRms>(hipStream_t, const GemvParams&, int, int, int, size_t);
}  // namespace prg
