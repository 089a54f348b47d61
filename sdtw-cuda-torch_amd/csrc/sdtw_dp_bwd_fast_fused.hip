// Instantiates the bwd wavefront kernels, fast arithmetic, fused cost (sdtw_dp.hpp).
#include "sdtw_dp.hpp"

namespace sdtw {
template hipError_t launch_dp_variant<true, false, true>(const DPParams&, bool, hipStream_t);
}  // namespace sdtw
