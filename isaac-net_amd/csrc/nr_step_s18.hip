// Step-kernel instantiations for 18 subbands (RBGs), one cell: HARQ processes 2, 4, 8, 16 x (IR combining) x
// (per-subband SNR input) with a runtime segment width, the plain case for 32-robot envs with the width fixed at compile
// time, and envs of 65..128 and 129..256 robots on two and four wavefronts.
#include "nr_step.h"

namespace inet {
StepFn pick_step_s18(int P, bool ir, bool vref, int rb, int fx) { return pick_step_s<18>(P, ir, vref, rb, fx); }
StepFn pick_step_w2_s18(int P, bool ir, int fx) { return pick_step_w2_s<18>(P, ir, fx); }
StepFn pick_step_w4_s18(int P, bool ir) { return pick_step_w4_s<18>(P, ir); }
}  // namespace inet

INET_PHASE_READER(inet_nr_phase_clocks_s18)
