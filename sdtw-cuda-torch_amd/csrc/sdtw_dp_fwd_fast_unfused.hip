// Instantiates the fwd wavefront kernels, fast arithmetic, unfused cost (sdtw_dp.hpp).
#include "sdtw_dp.hpp"

namespace sdtw {
template hipError_t launch_dp_variant<false, false, false>(const DPParams&, bool, hipStream_t);
}  // namespace sdtw
