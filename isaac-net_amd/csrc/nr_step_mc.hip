// Step-kernel instantiations for several cells per env (NRNet.step_cells): 3 cells, 8 / 13 / 14 subbands (RBGs),
// HARQ processes 2, 4, 8, 16 x (IR combining), pose input, runtime segment width.
#include "nr_step.h"

namespace inet {
StepFn pick_step_mc(int S, int C, int P, bool ir) {
    if (C != 3) return nullptr;
    if (S == 8) return pick_step_mc_s<8>(P, ir);
    if (S == 13) return pick_step_mc_s<13>(P, ir);
    if (S == 14) return pick_step_mc_s<14>(P, ir);
    return nullptr;
}
}  // namespace inet
