// q8_gemv_fma.hip -- the decode GEMVs with the SDOT paths' fma epilogue
// acc = fma(f32(I), sa*dw, acc) (Q8Decode.cpp:192-203), instantiated apart
// from the scalar ones so that the two sets compile in parallel.
#include "q8_gemv.h"

namespace llmcp_q8 {

hipError_t launch_gemv_fma(const GemvArgs &a, const GemvLaunch &l, bool in_wg,
                           hipStream_t s) {
  return in_wg ? launch_gemv_in<IN_WG, true>(a, l, s)
               : launch_gemv_in<IN_PRE, true>(a, l, s);
}

hipError_t launch_gemv_group_fma(const GemvGroupArgs &a, const GemvLaunch &l,
                                 hipStream_t s) {
  return launch_gemv_group<true>(a, l, s);
}

}  // namespace llmcp_q8
