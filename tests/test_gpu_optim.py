"""repo_amd.optim.Adam (one HIP launch per step) against torch.optim.Adam, the
optimizer the reference builds (gaussian_trace/model.py:172-189), run in
float64 on the CPU."""
from __future__ import annotations

import io

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


# ---------------------------------------------------------------- Adan
# repo_amd.optim.Adan / adan_step_from_grad_tilelang against the oracle's
# float64 restatement of ops/optim.py:78-110 (oracle.adan_step64), each step
# started from the device's own fp32 state.


def _adan_ref_step(p, g, st, *, step, lr, betas, eps, wd, no_prox, clip):
    from oracle import oracle as O
    c = lambda t: t.detach().cpu().double().numpy()  # noqa: E731
    return O.adan_step64(c(p), c(g), c(st["exp_avg"]), c(st["exp_avg_sq"]),
                         c(st["exp_avg_diff"]), c(st["neg_pre_grad"]), step=step, lr=lr,
                         betas=betas, eps=eps, weight_decay=wd, no_prox=no_prox, clip=clip)


def _check_adan(p_old, p_new, st, ref, tag):
    """p per element within 1e-6 |p| + 1e-5 |update| (fp32 rounding of p and
    of the update); states within 1e-5 relative plus 1e-6 of their largest
    magnitude."""
    import numpy as np
    rp, rm, rn, rd, rnpg = ref
    got = p_new.detach().cpu().double().numpy()
    old = p_old.cpu().double().numpy()
    err = np.abs(got - rp)
    tol = 1e-6 * np.abs(old) + 1e-5 * np.abs(rp - old) + 1e-12
    assert np.all(err <= tol), (tag, "param", float((err - tol).max()))
    for name, r in (("exp_avg", rm), ("exp_avg_sq", rn), ("exp_avg_diff", rd),
                    ("neg_pre_grad", rnpg)):
        x = st[name].cpu().double().numpy()
        bound = 1e-5 * np.abs(r) + 1e-6 * max(np.abs(r).max(), 1e-30)
        assert np.all(np.abs(x - r) <= bound), (tag, name, float(np.abs(x - r).max()))


@pytest.mark.gpu
@pytest.mark.parametrize("no_prox", [False, True])
@pytest.mark.parametrize("max_grad_norm", [0.0, 0.5])
def test_adan_matches_oracle(no_prox, max_grad_norm):
    import numpy as np
    from repo_amd.optim import Adan
    base = _params(1)
    ours = [p.clone().cuda().requires_grad_(True) for p in base]
    groups = [{"params": [ours[0]], "lr": 2e-2, "weight_decay": 0.02},
              {"params": [ours[1], ours[2]], "lr": 1e-1, "betas": (0.9, 0.8, 0.95)}]
    opt = Adan(groups, lr=1e-3, eps=1e-8, max_grad_norm=max_grad_norm, no_prox=no_prox)
    for step in range(1, 6):
        gs = _grads(base, step)
        for p, g in zip(ours, gs):
            p.grad = g.cuda()
        clip = 1.0
        if max_grad_norm > 0:
            norm = float(np.sqrt(sum(float((g.double() ** 2).sum()) for g in gs)))
            clip = min(max_grad_norm / (norm + 1e-8), 1.0)
            assert clip < 1.0
        before = [(p.detach().clone(), {k: v.clone() for k, v in opt.state[p].items()}
                   if opt.state[p] else None) for p in ours]
        opt.step()
        for gi, group in enumerate(opt.param_groups):
            assert group["step"] == step
            for p in group["params"]:
                k = next(i for i, q in enumerate(ours) if q is p)
                p_old, st_old = before[k]
                if st_old is None:
                    st_old = {n: torch.zeros_like(p) for n in
                              ("exp_avg", "exp_avg_sq", "exp_avg_diff", "neg_pre_grad")}
                ref = _adan_ref_step(p_old, gs[k], st_old, step=step, lr=group["lr"],
                                     betas=group["betas"], eps=group["eps"],
                                     wd=group["weight_decay"], no_prox=no_prox, clip=clip)
                _check_adan(p_old, p, opt.state[p], ref, (step, k))


@pytest.mark.gpu
def test_adan_functional_form_matches_oracle():
    """adan_step_from_grad_tilelang on a non-contiguous gradient with an
    explicit clip factor, three steps."""
    from repo_amd.optim import adan_step_from_grad_tilelang
    g0 = torch.Generator().manual_seed(5)
    p = torch.randn((64, 33), generator=g0).cuda()
    st = {n: torch.zeros_like(p) for n in
          ("exp_avg", "exp_avg_sq", "exp_avg_diff", "neg_pre_grad")}
    kw = dict(lr=0.05, betas=(0.98, 0.92, 0.99), eps=1e-8, weight_decay=0.1, no_prox=False)
    for step in (1, 2, 3):
        g = torch.randn((33, 64), generator=g0).cuda().t()
        assert not g.is_contiguous()
        p_old = p.clone()
        st_old = {k: v.clone() for k, v in st.items()}
        adan_step_from_grad_tilelang(p, g, st["exp_avg"], st["exp_avg_sq"], st["exp_avg_diff"],
                                     st["neg_pre_grad"], step=step, clip_global_grad_norm=0.7,
                                     **kw)
        ref = _adan_ref_step(p_old, g, st_old, step=step, wd=kw["weight_decay"],
                             **{k: v for k, v in kw.items() if k != "weight_decay"}, clip=0.7)
        _check_adan(p_old, p, st, ref, step)


@pytest.mark.gpu
def test_adan_first_step_closed_form_and_many_tensors():
    """Step 1 moves every element by lr g / (|g| + eps) whatever the betas
    (to fp32 rounding of the bias corrections); 20 tensors span two launches;
    a parameter without a gradient is left alone and gets no state."""
    from repo_amd.optim import Adan
    ps = [torch.full((5 + k,), float(k), device="cuda", requires_grad=True) for k in range(20)]
    opt = Adan(ps, lr=0.25, eps=0.0)
    for k, p in enumerate(ps):
        p.grad = None if k == 7 else torch.full_like(p, -2.0 if k % 2 else 3.0)
    opt.step()
    for k, p in enumerate(ps):
        want = float(k) if k == 7 else float(k) + (0.25 if k % 2 else -0.25)
        assert torch.allclose(p.detach(), torch.full_like(p, want), rtol=0, atol=1e-6), k
    assert len(opt.state[ps[7]]) == 0


@pytest.mark.gpu
def test_adan_state_dict_round_trip_and_restart():
    """A state_dict loaded into a fresh Adan continues bit for bit like the
    original; restart_opt zeroes the states and the step count."""
    from repo_amd.optim import Adan
    base = _params(2)
    a = [p.clone().cuda().requires_grad_(True) for p in base]
    opt = Adan(a, lr=1e-2, weight_decay=0.01, max_grad_norm=1.0)
    for step in range(3):
        for p, g in zip(a, _grads(base, step)):
            p.grad = g.cuda()
        opt.step()
    b = [p.detach().clone().requires_grad_(True) for p in a]
    opt_b = Adan(b, lr=1e-2, weight_decay=0.01, max_grad_norm=1.0)
    # Through a serialized checkpoint: load_state_dict keeps the very tensors
    # it is given when dtype and device already match.
    buf = io.BytesIO()
    torch.save(opt.state_dict(), buf)
    buf.seek(0)
    opt_b.load_state_dict(torch.load(buf, weights_only=True))
    for o, ps in ((opt, a), (opt_b, b)):
        for p, g in zip(ps, _grads(base, 9)):
            p.grad = g.cuda()
        o.step()
    for p, q in zip(a, b):
        assert torch.equal(p, q)
        for k in ("exp_avg", "exp_avg_sq", "exp_avg_diff", "neg_pre_grad"):
            assert torch.equal(opt.state[p][k], opt_b.state[q][k])
    assert opt_b.param_groups[0]["step"] == 4
    opt.restart_opt()
    assert opt.param_groups[0]["step"] == 0
    assert all(float(v.abs().sum()) == 0.0 for p in a for v in opt.state[p].values())


def test_adan_constructor_checks_and_host_tensors():
    """The reference's argument checks (manbo/optim.py:24-37), and host
    parameters refused before any work."""
    from repo_amd.optim import Adan
    p = [torch.zeros(3, requires_grad=True)]
    for kw in (dict(lr=-1.0), dict(eps=-1.0), dict(max_grad_norm=-1.0),
               dict(betas=(1.0, 0.9, 0.9)), dict(betas=(0.9, -0.1, 0.9)),
               dict(betas=(0.9, 0.9, 1.0)), dict(tilelang_threads=0)):
        with pytest.raises(ValueError):
            Adan(p, **kw)
    opt = Adan(p)
    assert opt.defaults["betas"] == (0.98, 0.92, 0.99) and opt.defaults["no_prox"] is False
    p[0].grad = torch.ones(3)
    with pytest.raises(ValueError, match="CUDA"):
        opt.step()
