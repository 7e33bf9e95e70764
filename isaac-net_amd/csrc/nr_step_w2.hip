// Step-kernel instantiations for envs of 65..128 robots (one env per workgroup of two wavefronts): 8 / 13 subbands
// (RBGs), HARQ processes 2, 4, 8, 16 x (IR combining), pose or SNR input; and config 5's switches fixed at compile
// time (8 RBGs, 8 HARQ, FX = 2).
#include "nr_step.h"

namespace inet {
StepFn pick_step_w2(int S, int P, bool ir, int fx) {
    if (S == 8) return pick_step_w2_s<8>(P, ir, fx);
    if (S == 13) return pick_step_w2_s<13>(P, ir, fx);
    return nullptr;
}
}  // namespace inet

INET_PHASE_READER(inet_nr_phase_clocks_w2)
