// Instantiates the fwd wavefront kernels, exact arithmetic, fused cost (sdtw_dp.hpp).
#include "sdtw_dp.hpp"

namespace sdtw {
template hipError_t launch_dp_variant<false, true, true>(const DPParams&, bool, hipStream_t);
}  // namespace sdtw
