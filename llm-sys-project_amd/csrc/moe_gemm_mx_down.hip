// Grouped GEMM kernel variants: <DT_MX, MODE_DOWN, packed> (MXFP4 weights).
#include "moe_gemm.hpp"

namespace amdmoe {

template int launch_gemm_variant<DT_MX, MODE_DOWN, true>(const GemmArgs&, long, hipStream_t);

}  // namespace amdmoe
