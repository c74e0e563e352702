// Q4 GEMV kernel variants: epilogue argmax.
#include "q4_gemv_launch.hpp"

namespace prg {
template int launch_m<kEpiArgmax, kNormNone>(hipStream_t, const GemvParams&, int, int, int, size_t);
}  // namespace prg
