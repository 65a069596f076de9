// Grouped GEMM kernel variants: <DT_FP8, MODE_UP, row-major>.
#include "moe_gemm.hpp"

namespace amdmoe {

template int launch_gemm_variant<DT_FP8, MODE_UP, false>(const GemmArgs&, long, hipStream_t);

}  // namespace amdmoe
