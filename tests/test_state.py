"""Checkpoint / state format of the FFI layer and its optimizer (SURVEY 8(f)4 row:
shared_ffi/rewire.py:110,115,127 keys, src/runner.py:304-334)."""
import io

import pytest
import torch

from haste_amd.optim_sr import SRSgd
from haste_amd.rewire import GroupFixedFanIn, inflate_group_locations


def test_layer_state_dict_keys_and_dtypes():
    """Keys, shapes and dtypes of the reference layer: weights [O, F] and bias [O]
    parameters, group_locations int32 [ceil(O/G), F] persistent buffer; a state
    dict loads into a fresh layer unchanged."""
    torch.manual_seed(0)
    layer = GroupFixedFanIn(300, 1001, 64, group_size=32, prune_mode="fraction", rewire_fraction=0.15,
                            dtype=torch.bfloat16)
    sd = layer.state_dict()
    assert list(sd) == ["weights", "bias", "group_locations"]
    assert sd["weights"].shape == (1001, 64) and sd["weights"].dtype == torch.bfloat16
    assert sd["bias"].shape == (1001,) and sd["bias"].dtype == torch.bfloat16
    assert sd["group_locations"].shape == (32, 64) and sd["group_locations"].dtype == torch.int32
    buf = io.BytesIO()
    torch.save(sd, buf)
    buf.seek(0)
    other = GroupFixedFanIn(300, 1001, 64, group_size=32, prune_mode="fraction", rewire_fraction=0.15,
                            dtype=torch.bfloat16)
    other.load_state_dict(torch.load(buf, weights_only=True))
    for k, v in other.state_dict().items():
        assert torch.equal(v, sd[k])


def test_inflate_group_locations():
    """Each group row repeated group_size times, truncated to L (src/runner.py:323-334)."""
    g = torch.arange(12, dtype=torch.int32).view(3, 4)
    out = inflate_group_locations(g, 7, 3)
    assert out.shape == (7, 4)
    for l in range(7):
        assert torch.equal(out[l], g[l // 3])


def test_optimizer_state_keeps_fp32_momentum_and_seed():
    """SRSgd.state_dict carries the current seed and the fp32 momentum buffer, and
    load_state_dict restores the buffer in fp32 (torch's default would cast it to
    the bf16 parameter dtype)."""
    p = torch.nn.Parameter(torch.zeros(10, dtype=torch.bfloat16))
    opt = SRSgd([p], lr=0.1, momentum=0.9, seed=77)
    m = torch.linspace(-1, 1, 10, dtype=torch.float32) / 3  # not representable in bf16
    opt.state[p]["momentum_buf"] = m.clone()
    opt.param_groups[0]["seed"] = 81
    buf = io.BytesIO()
    torch.save(opt.state_dict(), buf)
    buf.seek(0)
    q = torch.nn.Parameter(torch.zeros(10, dtype=torch.bfloat16))
    opt2 = SRSgd([q], lr=0.1, momentum=0.9, seed=5)
    opt2.load_state_dict(torch.load(buf, weights_only=True))
    assert opt2.param_groups[0]["seed"] == 81
    mb = opt2.state[q]["momentum_buf"]
    assert mb.dtype == torch.float32 and torch.equal(mb, m)


def test_momentum_buffers_always_in_state():
    """As the reference's SRSgd.__init__ (shared_ffi/optim_sr.py:35-44), every
    parameter that requires a gradient has a zero fp32 momentum_buf from the
    start, also with momentum 0, so a checkpoint has the state keys that the
    reference's step reads unconditionally (optim_sr.py:70)."""
    p = torch.nn.Parameter(torch.zeros(6, 4, dtype=torch.bfloat16))
    b = torch.nn.Parameter(torch.zeros(6, dtype=torch.bfloat16))
    frozen = torch.nn.Parameter(torch.zeros(3), requires_grad=False)
    opt = SRSgd([p, b, frozen], lr=0.1, momentum=0.0, seed=1)
    sd = opt.state_dict()
    assert set(sd["state"]) == {0, 1}
    for i, t in ((0, p), (1, b)):
        m = sd["state"][i]["momentum_buf"]
        assert m.dtype == torch.float32 and m.shape == t.shape and not m.any()
    # a reference-shaped consumer: every listed parameter's state has the key
    buf = io.BytesIO()
    torch.save(sd, buf)
    buf.seek(0)
    loaded = torch.load(buf, weights_only=True)
    for i in loaded["param_groups"][0]["params"][:2]:
        assert "momentum_buf" in loaded["state"][i]


def test_zero_grad_matches_torch_optimizer():
    """SRSgd.zero_grad does what torch.optim.Optimizer.zero_grad does: grads set
    to None by default, or detached and zeroed in place with set_to_none=False."""
    for set_to_none in (True, False):
        ps = [torch.nn.Parameter(torch.randn(3, 4)), torch.nn.Parameter(torch.randn(5))]
        qs = [torch.nn.Parameter(p.detach().clone()) for p in ps]
        for a, b in zip(ps, qs):
            a.grad = torch.randn_like(a)
            b.grad = a.grad.clone()
        qs[1].grad = None
        ps[1].grad = None
        SRSgd(ps, lr=0.1).zero_grad(set_to_none=set_to_none)
        torch.optim.SGD(qs, lr=0.1).zero_grad(set_to_none=set_to_none)
        for a, b in zip(ps, qs):
            assert (a.grad is None) == (b.grad is None)
            if a.grad is not None:
                assert torch.equal(a.grad, b.grad) and not a.grad.requires_grad


def test_step_hooks_match_torch_optimizer():
    """SRSgd.step runs without torch's profiler wrapper but keeps its hook
    semantics: global then per-optimizer pre-hooks (which may replace the
    arguments), then per-optimizer then global post-hooks, each given the
    optimizer and (optimizer, closure) as args; the closure's loss is returned.
    torch.optim.SGD, which torch wraps, is the yardstick (fp32 parameters take
    SRSgd's torch path, so this runs on the CPU)."""
    from torch.optim.optimizer import (register_optimizer_step_post_hook,
                                       register_optimizer_step_pre_hook)

    def run(make):
        calls = []
        p = torch.nn.Parameter(torch.ones(3))
        p.grad = torch.full((3,), 2.0)
        opt = make([p])
        opt.register_step_pre_hook(lambda o, a, k: calls.append(("pre", o is opt, len(a))))
        opt.register_step_post_hook(lambda o, a, k: calls.append(("post", o is opt, len(a))))

        def swap_closure(o, a, k):
            if o is opt:
                calls.append(("swap",))
                return (a[0], lambda: torch.tensor(7.0)), k

        handles = [register_optimizer_step_pre_hook(lambda o, a, k: calls.append(("gpre", o is opt))),
                   register_optimizer_step_pre_hook(swap_closure),
                   register_optimizer_step_post_hook(lambda o, a, k: calls.append(("gpost", o is opt)))]
        try:
            loss = opt.step(lambda: torch.tensor(1.0))
        finally:
            for h in handles:
                h.remove()
        return calls, loss, p.detach().clone()

    mine = run(lambda ps: SRSgd(ps, lr=0.5, momentum=0.0))
    ref = run(lambda ps: torch.optim.SGD(ps, lr=0.5))
    assert mine[0] == ref[0]
    assert float(mine[1]) == float(ref[1]) == 7.0
    assert torch.equal(mine[2], ref[2])
    assert type(SRSgd([torch.nn.Parameter(torch.ones(1))])).step is SRSgd.__dict__["step"]


@pytest.mark.gpu
def test_resume_is_bit_identical(dev):
    """Train, checkpoint layer + optimizer, keep training; a fresh layer and
    optimizer loaded from the checkpoint produce the same weights bit for bit."""
    B, D, O, G, F = 32, 256, 2000, 32, 64

    def make():
        torch.manual_seed(0)
        layer = GroupFixedFanIn(D, O, F, group_size=G, prune_mode="fraction", rewire_fraction=0.15,
                                dtype=torch.bfloat16).to(dev)
        return layer, SRSgd(layer.parameters(), lr=0.05, weight_decay=1e-4, momentum=0.9, seed=42)

    def train(layer, opt, k, seed):
        g = torch.Generator().manual_seed(seed)
        for _ in range(k):
            x = torch.randn(B, D, generator=g).to(torch.bfloat16).to(dev)
            dY = (torch.randn(B, O, generator=g) * 0.1).to(torch.bfloat16).to(dev)
            opt.zero_grad()
            layer(x).backward(dY)
            opt.step()

    layer, opt = make()
    train(layer, opt, 3, seed=1)
    ck = io.BytesIO()
    torch.save({"state_dict": layer.state_dict(), "optimizer": opt.state_dict()}, ck)
    train(layer, opt, 2, seed=2)
    ck.seek(0)
    st = torch.load(ck, weights_only=True)
    layer2, opt2 = make()
    layer2.load_state_dict(st["state_dict"])
    opt2.load_state_dict(st["optimizer"])
    train(layer2, opt2, 2, seed=2)
    torch.cuda.synchronize()
    for a, b in zip(layer.state_dict().values(), layer2.state_dict().values()):
        assert torch.equal(a, b)
