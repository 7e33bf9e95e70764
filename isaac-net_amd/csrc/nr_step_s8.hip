// Step-kernel instantiations for 8 subbands (RBGs): HARQ processes 2, 4, 8, 16 x (IR combining) x (per-subband
// SNR input), with a runtime segment width; and the plain case (no IR, pose or SNR input) for 32-robot envs with the
// segment width fixed at compile time.
#include "nr_step.h"

namespace inet {
StepFn pick_step_s8(int P, bool ir, bool vref, int rb, int fx) { return pick_step_s<8>(P, ir, vref, rb, fx); }
}  // namespace inet

INET_PHASE_READER(inet_nr_phase_clocks_s8)
