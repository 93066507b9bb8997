"""repo_amd.optim.Adam (one HIP launch per step) against torch.optim.Adam, the
optimizer the reference builds (gaussian_trace/model.py:172-189), run in
float64 on the CPU."""
from __future__ import annotations

import pytest
import torch


def _params(seed):
    g = torch.Generator().manual_seed(seed)
    cub = torch.randn((1000, 4, 2), generator=g)
    col = torch.rand((333, 3), generator=g)
    opa = torch.rand((333,), generator=g)
    return [cub, col, opa]


def _grads(params, step):
    g = torch.Generator().manual_seed(100 + step)
    return [torch.randn(p.shape, generator=g) * (1e-3 if k == 0 else 1.0)
            for k, p in enumerate(params)]


@pytest.mark.gpu
@pytest.mark.parametrize("weight_decay", [0.0, 0.01])
def test_adam_matches_torch_adam(weight_decay):
    from repo_amd.optim import Adam
    base = _params(0)
    ours = [p.clone().cuda().requires_grad_(True) for p in base]
    ref = [p.clone().double().requires_grad_(True) for p in base]
    groups = lambda ps: [{"params": [ps[0]], "lr": 2e-2},  # noqa: E731
                         {"params": [ps[1], ps[2]], "lr": 1e-1}]
    opt = Adam(groups(ours), lr=1e-3, weight_decay=weight_decay)
    opt_ref = torch.optim.Adam(groups(ref), lr=1e-3, weight_decay=weight_decay, foreach=False)
    for step in range(4):
        gs = _grads(base, step)
        for p, q, g in zip(ours, ref, gs):
            p.grad = g.cuda()
            q.grad = g.double()
        opt.step()
        opt_ref.step()
        for p, q in zip(ours, ref):
            err = (p.detach().cpu().double() - q.detach()).abs().max().item()
            assert err <= 2e-6 * max(1.0, q.detach().abs().max().item()), (step, err)
    for p, q in zip(ours, ref):
        s, r = opt.state[p], opt_ref.state[q]
        assert float(s["step"]) == float(r["step"]) == 4.0
        for k in ("exp_avg", "exp_avg_sq"):
            err = (s[k].cpu().double() - r[k]).abs().max().item()
            assert err <= 1e-5 * max(r[k].abs().max().item(), 1e-30), (k, err)


@pytest.mark.gpu
def test_adam_skips_params_without_grad_and_many_tensors():
    from repo_amd.optim import Adam
    ps = [torch.full((7 + k,), float(k), device="cuda", requires_grad=True) for k in range(20)]
    opt = Adam(ps, lr=0.5)
    for k, p in enumerate(ps):
        p.grad = None if k == 3 else torch.ones_like(p)
    opt.step()
    for k, p in enumerate(ps):
        want = float(k) if k == 3 else float(k) - 0.5  # first step moves by lr * sign(g)
        assert torch.allclose(p.detach(), torch.full_like(p, want), atol=1e-6), k
    assert len(opt.state[ps[3]]) == 0


def test_adam_rejects_unsupported_options():
    from repo_amd.optim import Adam
    p = [torch.zeros(3, requires_grad=True)]
    with pytest.raises(NotImplementedError):
        Adam(p, amsgrad=True)
    with pytest.raises(ValueError):
        Adam(p, lr=-1.0)


@pytest.mark.gpu
def test_adam_runs_step_hooks_and_state_dict_round_trips():
    from repo_amd.optim import Adam
    p = torch.zeros(5, device="cuda", requires_grad=True)
    opt = Adam([p], lr=0.1)
    seen = []
    h1 = opt.register_step_pre_hook(lambda o, a, k: seen.append("pre"))
    h2 = opt.register_step_post_hook(lambda o, a, k: seen.append("post"))
    p.grad = torch.ones_like(p)
    opt.step()
    assert seen == ["pre", "post"]
    h1.remove()
    h2.remove()
    sd = opt.state_dict()
    q = torch.zeros(5, device="cuda", requires_grad=True)
    ref = torch.optim.Adam([q], lr=0.1)
    ref.load_state_dict(sd)
    assert float(ref.state[q]["step"]) == 1.0
    assert torch.equal(ref.state[q]["exp_avg"], opt.state[p]["exp_avg"])
