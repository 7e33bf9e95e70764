// Step-kernel instantiations for envs of 65..128 robots (one env per workgroup of two wavefronts): 8 / 13 subbands
// (RBGs), HARQ processes 2, 4, 8, 16 x (IR combining), pose or SNR input.
#include "nr_step.h"

namespace inet {
StepFn pick_step_w2(int S, int P, bool ir) {
    if (S == 8) return pick_step_w2_s<8>(P, ir);
    if (S == 13) return pick_step_w2_s<13>(P, ir);
    return nullptr;
}
}  // namespace inet
