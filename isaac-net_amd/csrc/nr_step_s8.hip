// Step-kernel instantiations for 8 subbands (RBGs): HARQ processes 2, 4, 8, 16 x (IR combining) x (per-subband
// SNR input).
#include "nr_step.h"

namespace inet {
StepFn pick_step_s8(int P, bool ir, bool vref) { return pick_step_s<8>(P, ir, vref); }
}  // namespace inet
