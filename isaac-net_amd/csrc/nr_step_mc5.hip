// Step-kernel instantiations for 5 cells per env (NRNet.step_cells; the hex sites of config.py:1417-1429):
// 8 / 13 / 14 subbands (RBGs), HARQ processes 2, 4, 8, 16 x (IR combining), pose input, runtime segment width.
#include "nr_step.h"

namespace inet {
StepFn pick_step_mc5(int S, int P, bool ir, int fx, int rb) {
    if (S == 8) return pick_step_mc_s<8, 5>(P, ir, fx, rb);
    if (S == 13) return pick_step_mc_s<13, 5>(P, ir, fx, rb);
    if (S == 14) return pick_step_mc_s<14, 5>(P, ir, fx, rb);
    return nullptr;
}
}  // namespace inet

INET_PHASE_READER(inet_nr_phase_clocks_mc5)
