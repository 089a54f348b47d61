// Instantiates the fused backward's gradient-mode kernels, fast arithmetic (sdtw_dp.hpp).
#include "sdtw_dp.hpp"

namespace sdtw {
template hipError_t launch_dp_grad<false>(const DPParams&, hipStream_t);
}  // namespace sdtw
