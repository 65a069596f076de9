// Grouped GEMM kernel variants: <DT_MX, MODE_UP, packed> (MXFP4 weights).
#include "moe_gemm.hpp"

namespace amdmoe {

template int launch_gemm_variant<DT_MX, MODE_UP, true>(const GemmArgs&, long, hipStream_t);

}  // namespace amdmoe
