// Step-kernel instantiations for several cells per env (NRNet.step_cells): 3 cells (2 and 4..7 cells in
// nr_step_mc<C>.hip), 8 / 13 / 14 subbands (RBGs), HARQ processes 2, 4, 8, 16 x (IR combining), pose input,
// runtime segment width; and config 3's switches fixed at compile time (14 RBGs, 8 HARQ, FX = 2) for 64-robot
// envs (segment width fixed at compile time).
#include "nr_step.h"

namespace inet {
StepFn pick_step_mc(int S, int C, int P, bool ir, int fx, int rb) {
    if (C == 2) return pick_step_mc2(S, P, ir, fx, rb);
    if (C == 4) return pick_step_mc4(S, P, ir, fx, rb);
    if (C == 5) return pick_step_mc5(S, P, ir, fx, rb);
    if (C == 6) return pick_step_mc6(S, P, ir, fx, rb);
    if (C == 7) return pick_step_mc7(S, P, ir, fx, rb);
    if (C != 3) return nullptr;
    if (S == 8) return pick_step_mc_s<8, 3>(P, ir, fx, rb);
    if (S == 13) return pick_step_mc_s<13, 3>(P, ir, fx, rb);
    if (S == 14) return pick_step_mc_s<14, 3>(P, ir, fx, rb);
    return nullptr;
}
}  // namespace inet

INET_PHASE_READER(inet_nr_phase_clocks_mc)
