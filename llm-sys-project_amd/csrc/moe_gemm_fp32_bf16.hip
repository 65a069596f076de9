// Grouped GEMM kernel variants: fp32 UP / DOWN (row-major weights), bf16 UP / DOWN (row-major and packed weights).
#include "moe_gemm.hpp"

namespace amdmoe {

template int launch_gemm_variant<DT_F32, MODE_UP, false>(const GemmArgs&, long, hipStream_t);
template int launch_gemm_variant<DT_F32, MODE_DOWN, false>(const GemmArgs&, long, hipStream_t);
template int launch_gemm_variant<DT_BF16, MODE_UP, false>(const GemmArgs&, long, hipStream_t);
template int launch_gemm_variant<DT_BF16, MODE_DOWN, false>(const GemmArgs&, long, hipStream_t);
template int launch_gemm_variant<DT_BF16, MODE_UP, true>(const GemmArgs&, long, hipStream_t);
template int launch_gemm_variant<DT_BF16, MODE_DOWN, true>(const GemmArgs&, long, hipStream_t);

}  // namespace amdmoe
