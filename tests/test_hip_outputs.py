"""Ownership of the step outputs (swarp/interop/autograd.py:229-296: the grad path is
functional with fresh outputs).  For a 2-D fleet the four drone fields are not stepped;
every returned state still owns them -- copies of the input's, so an in-place edit of an
input or of one output shows nowhere else -- and their gradient passes through to the
input unchanged.  The trajectory is built on first use and matches the final state."""

import pytest
import torch

from cases import nav_agents, nav_world
from hip_helpers import make_stepper
from swarp_amd import TorchState, rollout, warp_step

pytestmark = pytest.mark.gpu
TAIL = ("z", "vz", "attitude", "body_rates")


def _state(E, A, grad_tail):
    g = torch.Generator(device="cpu").manual_seed(3)
    c = lambda t: t.cuda()  # noqa: E731
    z = torch.zeros(E, A)
    tail = [c(torch.rand(E, A, generator=g)), c(torch.rand(E, A, generator=g)),
            c(torch.rand(E, A, 4, generator=g)), c(torch.rand(E, A, 3, generator=g))]
    if grad_tail:
        tail = [t.requires_grad_(True) for t in tail]
    return TorchState(c(torch.rand(E, A, 2, generator=g) - 0.5).requires_grad_(True), c(z.clone()),
                      c(torch.zeros(E, A, 2)), c(z.clone()), c(z.clone()), *tail)


def test_rollout_outputs_own_drone_fields_and_pass_their_gradient():
    E, A, T = 6, 4, 5
    st = make_stepper(nav_agents(A), nav_world(A), 0.05, 2, torch.float32)
    s0 = _state(E, A, True)
    acts = (torch.rand(T, E, A, 2, device="cuda") * 2 - 1).requires_grad_(True)
    final, traj = rollout(st, s0, acts)
    assert len(traj) == T and traj[-1] is final
    ptrs = set()
    for s in traj:
        for name in TAIL:
            t, x = getattr(s, name), getattr(s0, name)
            assert torch.equal(t, x) and t.data_ptr() != x.data_ptr()
            ptrs.add(t.data_ptr())
    assert len(ptrs) == T * len(TAIL)  # no two states share a field
    before = final.z.clone()
    with torch.no_grad():
        s0.z.add_(1.0)
    assert torch.equal(final.z, before)
    w = [torch.rand_like(getattr(final, n)) for n in TAIL]
    loss = sum((wk * getattr(final, n)).sum() for wk, n in zip(w, TAIL)) + final.pos.sum()
    loss = loss + (traj[1].z * 2.0).sum()
    loss.backward()
    assert torch.allclose(s0.z.grad, w[0] + 2.0)
    for wk, n in zip(w[1:], TAIL[1:]):
        assert torch.equal(getattr(s0, n).grad, wk)


def test_warp_step_outputs_own_drone_fields():
    E, A = 5, 4
    st = make_stepper(nav_agents(A), nav_world(A), 0.05, 1, torch.float32)
    s0 = _state(E, A, False)
    a = (torch.rand(E, A, 2, device="cuda") * 2 - 1).requires_grad_(True)
    out = warp_step(st, s0, a)
    for name in TAIL:
        t, x = getattr(out, name), getattr(s0, name)
        assert torch.equal(t, x) and t.data_ptr() != x.data_ptr()


def test_trajectory_matches_final_and_defaults():
    """Omitted drone fields: zeros and the identity attitude in every returned state."""
    E, A, T = 4, 4, 3
    st = make_stepper(nav_agents(A), nav_world(A), 0.05, 1, torch.float32)
    pos = (torch.rand(E, A, 2, device="cuda") - 0.5).requires_grad_(True)
    acts = torch.rand(T, E, A, 2, device="cuda") * 2 - 1
    z = torch.zeros(E, A, device="cuda")
    final, traj = rollout(st, TorchState(pos, z.clone(), torch.zeros(E, A, 2, device="cuda"),
                                         z.clone(), z.clone()), acts)
    ident = torch.zeros(E, A, 4, device="cuda")
    ident[..., 3] = 1.0
    for s in traj:
        assert torch.equal(s.attitude, ident) and torch.equal(s.z, torch.zeros(E, A, device="cuda"))
    assert torch.equal(traj[-1].pos, final.pos)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("E,A", [(3, 5), (1, 1), (16000, 16)])
def test_fill_state_defaults_on_device_equals_the_host_defaults(E, A, dtype):
    """swarp_state_defaults (one launch) writes what the host path builds with torch:
    zeros and the identity quaternion, for sizes whose 9 E A elements are not a multiple
    of the four elements a lane writes; fields the caller gave are kept."""
    from swarp_amd.autograd import fill_state_defaults

    def defaults(dev):
        pos = torch.zeros(E, A, 2, device=dev, dtype=dtype)
        z = torch.zeros(E, A, device=dev, dtype=dtype)
        return fill_state_defaults(TorchState(pos, z, torch.zeros(E, A, 2, device=dev, dtype=dtype),
                                              z, z))

    got, want = defaults("cuda"), defaults("cpu")
    for name in TAIL:
        g, w = getattr(got, name), getattr(want, name)
        assert g.dtype == dtype and g.shape == w.shape and torch.equal(g.cpu(), w)
    assert torch.equal(want.attitude[..., 3], torch.ones(E, A, dtype=dtype))
    vz = torch.full((E, A), 7.0, device="cuda", dtype=dtype)
    pos = torch.zeros(E, A, 2, device="cuda", dtype=dtype)
    s = fill_state_defaults(TorchState(pos, pos[..., 0], pos, pos[..., 0], pos[..., 0], vz=vz))
    assert s.vz is vz and torch.equal(s.z.cpu(), torch.zeros(E, A, dtype=dtype))
