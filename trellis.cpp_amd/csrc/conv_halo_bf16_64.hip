// LDS-staged MFMA conv: the bf16 features / 64-output-channel-tile instantiations.
#include "conv_halo_kernel.hpp"

namespace tsp {

int halo_launch_bf16_64(TSP_HALO_LAUNCH_ARGS) {
    return launch_out<true, 64>(odt, planned, feats, n, ci, nbr, plan, weight, bias, co, out, s,
                                     osc, skip, pad, ln, tr);
}

}  // namespace tsp
