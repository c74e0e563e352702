// Q4 GEMV kernel variants: epilogue plain.
#include "q4_gemv_launch.hpp"

namespace prg {
template int launch_m<kEpiPlain, kNormNone>(hipStream_t, const GemvParams&, int, int, int, size_t);
}  // namespace prg
