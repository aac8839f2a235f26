"""A training step captured once in a HIP graph (torch.cuda.graph) and replayed:
FFITrainStep(device_seed=True) reads the SR-SGD seed from device memory and
advances it there (haste_ffi_bwd_weights_sgd_dx_dev_seed), so each replay is the
next step of the seed += 1 schedule (shared_ffi/optim_sr.py:59-62).  Checked
bit for bit against the same steps run eagerly with host seeds: logits, dX and
the updated weights and bias after every replay (the eager program's own work
and a synchronisation between replays)."""
import numpy as np
import pytest
import torch

from haste_amd.step import FFITrainStep

pytestmark = pytest.mark.gpu


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("B,D,O,G,F", [(128, 256, 4100, 64, 64), (64, 768, 4096, 32, 32)])
def test_graph_replayed_step_matches_eager(dev, B, D, O, G, F):
    g = torch.Generator(device=dev).manual_seed(B + O)
    Gc = (O + G - 1) // G
    x = torch.randn(B, D, generator=g, device=dev).to(torch.bfloat16)
    W = ((torch.rand(O, F, generator=g, device=dev) * 2 - 1) / F ** 0.5).to(torch.bfloat16)
    bias = (torch.randn(O, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    idx = torch.randint(0, D, (Gc, F), generator=g, device=dev, dtype=torch.int32)
    Wg, bg = W.clone(), bias.clone()
    eager = FFITrainStep(W, bias, idx, B, D, G, 0.05, 1e-4, seed=42)
    graphed = FFITrainStep(Wg, bg, idx, B, D, G, 0.05, 1e-4, seed=42, device_seed=True)
    dY = torch.zeros(B, eager.ldo, dtype=torch.bfloat16, device=dev)
    dY[:, :O] = (torch.randn(B, O, generator=g, device=dev) * 0.1).to(torch.bfloat16)

    # one eager step each (the index plan is built here), then capture
    eager.step(x, dY, eager.ldo)
    graphed.step(x, dY, graphed.ldo)
    torch.cuda.synchronize()
    assert np.array_equal(bits(Wg), bits(W)) and graphed.current_seed() == 43
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        graphed.step(x, dY, graphed.ldo)
    torch.cuda.synchronize()
    assert graphed.current_seed() == 43  # capture runs nothing
    for k in range(4):
        eager.step(x, dY, eager.ldo)
        graph.replay()
        torch.cuda.synchronize()
        assert graphed.current_seed() == 44 + k
        assert np.array_equal(bits(graphed.logits), bits(eager.logits)), k
        assert np.array_equal(bits(graphed.dX), bits(eager.dX)), k
        assert np.array_equal(bits(Wg), bits(W)), k
        assert np.array_equal(bits(bg), bits(bias)), k
    assert eager.seed == graphed.current_seed() == 47


def test_device_seed_state_round_trip(dev):
    B, D, O, G, F = 64, 256, 1000, 32, 32
    W = torch.zeros(O, F, dtype=torch.bfloat16, device=dev)
    idx = torch.zeros((O + G - 1) // G, F, dtype=torch.int32, device=dev)
    st = FFITrainStep(W, None, idx, B, D, G, 0.05, 0.0, seed=7, device_seed=True)
    assert st.state_dict() == {"seed": 7}
    st.load_state_dict({"seed": 123})
    assert st.current_seed() == 123
    with pytest.raises(ValueError, match="defer_dx"):
        st.backward_weights_sgd(torch.zeros(B, st.ldo, dtype=torch.bfloat16, device=dev), st.ldo)
