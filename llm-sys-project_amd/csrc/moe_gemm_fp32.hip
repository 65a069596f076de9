// Grouped GEMM kernel variants: fp32 UP / DOWN (row-major weights).  The bf16
// GEMMs run grouped_gemm_bf16_w4_kernel (moe_gemm_bf16_w4.hip).
#include "moe_gemm.hpp"

namespace amdmoe {

template int launch_gemm_variant<DT_F32, MODE_UP, false>(const GemmArgs&, long, hipStream_t);
template int launch_gemm_variant<DT_F32, MODE_DOWN, false>(const GemmArgs&, long, hipStream_t);

}  // namespace amdmoe
