// Grouped GEMM kernel variants: <DT_F32, MODE_UP, row-major>, <DT_F32, MODE_DOWN, row-major>, <DT_BF16, MODE_UP, row-major>, <DT_BF16, MODE_DOWN, row-major>.
#include "moe_gemm.hpp"

namespace amdmoe {

template int launch_gemm_variant<DT_F32, MODE_UP, false>(const GemmArgs&, long, hipStream_t);
template int launch_gemm_variant<DT_F32, MODE_DOWN, false>(const GemmArgs&, long, hipStream_t);
template int launch_gemm_variant<DT_BF16, MODE_UP, false>(const GemmArgs&, long, hipStream_t);
template int launch_gemm_variant<DT_BF16, MODE_DOWN, false>(const GemmArgs&, long, hipStream_t);

}  // namespace amdmoe
