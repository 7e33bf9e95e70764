"""HIP engine vs the reference trajectories (tests/golden/, bitwise equal to the oracle by test_oracle_golden):
teacher-forced (the reference state is loaded before every step) and free running from the same seed. Integer state
and integer outputs must be bit-exact; float tolerances are those of gpu_util (float outputs 1e-5 relative)."""
import numpy as np
import pytest
import torch

from conftest import CASES, DL_CASES, MC_CASES
import gpu_util
from gpu_util import compare, load, set_radio_bound, teacher_forced
from oracle import replay
import isaac_net_amd as P

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", CASES + DL_CASES + MC_CASES)
def test_teacher_forced_bit_exact(name):
    print(f"case {name} teacher-forced", flush=True)
    n_bad, n, keys_i, keys_f = teacher_forced(P, name)
    print(f"{name}: integer flips {n_bad}/{n} robot-steps; float keys out of tolerance {keys_f}; max |deviation| "
          f"{ {k: f'{v:.2e}' for k, v in gpu_util.MAX_DEV.items()} }", flush=True)
    gpu_util.MAX_DEV.clear()
    assert n_bad == 0 and not keys_i, keys_i
    assert not keys_f, keys_f


@pytest.mark.parametrize("name", CASES + DL_CASES + MC_CASES)
def test_free_running_bit_exact(name):
    print(f"case {name} free running", flush=True)
    ref, cfgd, kind = load(name)
    cfg = P.NRConfig(**cfgd, seed=0)
    E, R = int(ref["E"]), int(ref["R"])
    eng = P.make_engine("L2", E, R, "cuda:0", cfg, seed=0)
    bad = []

    def on_step(s, o, acc):
        if int(ref[f"s{s:03d}/n_submit"]):
            mine = np.stack([a.cpu().numpy() for a in acc])
            if not np.array_equal(mine, ref[f"s{s:03d}/accepted"]):
                bad.append((s, "accepted"))
        set_radio_bound(ref, s, cfg, eng, kind)
        bi, bf, _ = compare(ref, s, o, eng.owner_state(), E, R)
        if bi or bf:
            bad.append((s, bi, bf))

    replay.run(eng, ref, kind, on_step=on_step, to=lambda a: torch.from_numpy(np.asarray(a)).to("cuda:0"))
    assert not bad, bad[:5]
    print(f"{name}: free running bit-exact; max |deviation| { {k: f'{v:.2e}' for k, v in gpu_util.MAX_DEV.items()} }",
          flush=True)
    gpu_util.MAX_DEV.clear()
    # counters: integer accumulators on the device vs the reference's float sums
    import json
    links = ("ul", "dl") if cfg.dl else ("ul",)
    for lk in links:
        want = json.loads(bytes(ref["counters_json"]))[lk]
        got = eng.counters()[lk]
        keys = ("tb_new", "tb_retx", "tb_ok", "tb_fail", "exhaust", "bytes_ok", "bytes_new", "lost_frames",
                "new_while_pending", "prb_used", "prb_avail")
        # with a 5G-LENA MAC switch on, the grant accounting too (mac.py:119-122)
        keys += tuple(k for k in ("tb_bytes", "tb_empty", "retx_block") if k in want)
        assert set(got) == set(want), (lk, sorted(set(got) ^ set(want)))
        for k in keys:
            assert got[k] == pytest.approx(want[k], rel=1e-6), (lk, k)
        assert got["ntx_hist"] == pytest.approx(want["ntx_hist"])
        assert got["rv_tx"] == pytest.approx(want["rv_tx"]) and got["rv_fail"] == pytest.approx(want["rv_fail"])


def test_reset_draws_match_reference_fields():
    """The device reset draws the shadowing fields of the reference (channels/fields.py draw_plane_waves) from the
    same counter-RNG uniforms: phases bitwise, wave vectors to two float32 ulp (cos / sin rounding, then the product with |k|)."""
    ref, cfgd, kind = load("c2")
    cfg = P.NRConfig(**cfgd, seed=0)
    eng = P.make_engine("L2", int(ref["E"]), int(ref["R"]), "cuda:0", cfg, seed=0)
    f = eng.st["field"][:, 0].cpu().numpy()
    for j, n in enumerate(("sf_los", "sf_nlos", "los_field")):
        k, phi = ref[f"s000/radio.{n}.k"][0], ref[f"s000/radio.{n}.phi"][0]
        assert np.array_equal(f[:, j, :, 2], phi)
        assert np.all(np.abs(f[:, j, :, :2] - k) <= 2 * np.spacing(np.abs(k).astype(np.float32))), n
