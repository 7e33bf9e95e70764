// Step-kernel instantiations for envs of 129..256 robots (one env per workgroup of four wavefronts): 8 / 13 subbands
// (RBGs; the other RBG counts' four-wavefront builds are in their nr_step_s<S>.hip units), HARQ processes 2, 4, 8, 16
// x (IR combining), pose or SNR input.
#include "nr_step.h"

namespace inet {
StepFn pick_step_w4(int S, int P, bool ir) {
    if (S == 8) return pick_step_w4_s<8>(P, ir);
    if (S == 13) return pick_step_w4_s<13>(P, ir);
#define INET_W4_S(SS) \
    if (S == SS) return pick_step_w4_s##SS(P, ir);
    INET_STEP_S_EXTRA(INET_W4_S)
#undef INET_W4_S
    return nullptr;
}
}  // namespace inet

INET_PHASE_READER(inet_nr_phase_clocks_w4)
