"""emprise_hip_delta_net_noalloc (the delta_net entry point that allocates nothing: its
scratch is a fixed device array) against emprise_hip_delta_net: outputs and states bit for
bit, on two calls in a row, the second with a smaller input, through the C ABI."""
import numpy as np
import pytest

from emprise_amd import DeltaNetParams, HipBackend, InvalidArgument

pytestmark = pytest.mark.gpu


def _gdn(be, rng, kh, vh, sd, cw):
    kd, vd = kh * sd, vh * sd
    ch = 2 * kd + vd
    prm = dict(conv=(rng.standard_normal(ch * cw) * 0.5).astype(np.float32),
               ssm_a=(-np.exp(rng.standard_normal(vh) * 0.5 - 2)).astype(np.float32),
               dt=(rng.standard_normal(vh) * 0.5 - 1).astype(np.float32),
               norm=(1 + 0.02 * rng.standard_normal(sd)).astype(np.float32))
    ws = [be.vector(prm[k]) for k in ("conv", "ssm_a", "dt", "norm")]
    ins = [be.to_device(rng.standard_normal(n).astype(np.float32)) for n in (ch, vd, vh, vh)]
    conv0 = (rng.standard_normal(ch * cw) * 0.3).astype(np.float32)
    rec0 = (rng.standard_normal(vh * sd * sd) * 0.05).astype(np.float32)
    states = []
    for _ in range(2):  # one pair of states per entry point, same start
        states.append((be.to_device(conv0), be.to_device(rec0), be.alloc(vd * 4)))
    ps = [DeltaNetParams(kh, vh, sd, cw, 1e-6, *ins, *ws, cs, rs, out) for cs, rs, out in states]
    return ps, states, (ch * cw, vh * sd * sd, vd)


def test_delta_net_noalloc_matches_delta_net():
    be = HipBackend(0)
    rng = np.random.default_rng(41)
    # the 9B shape (8192 channels), then a smaller one (1024 channels): the second call
    # reuses the scratch that the first one filled past its own width
    for kh, vh, sd, cw in ((16, 32, 128, 4), (4, 8, 64, 4)):
        ps, states, (nc, nr, nv) = _gdn(be, rng, kh, vh, sd, cw)
        for _ in range(2):  # two steps: the state carries over
            be.delta_net(ps[0])
            be.delta_net_noalloc(ps[1])
        (ca, ra, oa), (cb, rb, ob) = states
        assert np.array_equal(be.download(oa, nv).view(np.uint32), be.download(ob, nv).view(np.uint32))
        assert np.array_equal(be.download(ra, nr).view(np.uint32), be.download(rb, nr).view(np.uint32))
        assert np.array_equal(be.download(ca, nc).view(np.uint32), be.download(cb, nc).view(np.uint32))
    # wider than the fixed scratch: rejected before anything is launched
    p = ps[1]
    p.key_heads, p.value_heads, p.state_dim = 64, 448, 128  # 73728 channels
    with pytest.raises(InvalidArgument):
        be.delta_net_noalloc(p)
    be.close()
