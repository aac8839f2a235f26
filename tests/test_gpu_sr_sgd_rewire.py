"""GPU bit-exactness of stochastic rounding, the fused SR-SGD step and rewire
against the CPU oracle (identical Philox seed/offset contract)."""
import math

import numpy as np
import pytest
import torch

import oracle
from haste_amd import _C, _lib

pytestmark = pytest.mark.gpu


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("n,offset0,seed", [(1, 0, 123), (1000, 0, 42), (393216, 0, 123),
                                            (4099, 5, 2**32 + 7), (77, 2**32 - 3, 1)])
def test_sr_round(dev, n, offset0, seed):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    x[: min(n, 4)] = [0.0, -0.0, np.inf, 1e-40][: min(n, 4)]
    xd = torch.from_numpy(x).to(dev)
    out = torch.empty(n, dtype=torch.bfloat16, device=dev)
    _lib.call("haste_sr_round_bf16", xd.data_ptr(), out.data_ptr(), n, seed, offset0, _C.stream_of(xd))
    assert np.array_equal(bits(out), oracle.sr_round_bf16(x, seed, offset0))


def test_sr_round_unaligned_view(dev):
    x = np.random.default_rng(9).standard_normal(1001).astype(np.float32)
    xd = torch.from_numpy(x).to(dev)[1:]
    out = torch.empty(1001, dtype=torch.bfloat16, device=dev)[1:]
    _lib.call("haste_sr_round_bf16", xd.data_ptr(), out.data_ptr(), 1000, 42, 0, _C.stream_of(xd))
    assert np.array_equal(bits(out), oracle.sr_round_bf16(x[1:], 42, 0))


def test_stochastic_rounding_api(dev):
    from haste_amd.sr_triton import stochastic_rounding
    x = torch.randn(512, 768, device=dev)
    out = torch.empty_like(x, dtype=torch.bfloat16)
    stochastic_rounding(x, out, 123)
    assert np.array_equal(bits(out), oracle.sr_round_bf16(x.cpu().numpy(), 123, 0))


GRAD_DTYPES = [torch.float32, torch.bfloat16, torch.float16]


@pytest.mark.parametrize("gdt", GRAD_DTYPES)
@pytest.mark.parametrize("use_mom,do_sr", [(False, True), (True, True), (False, False), (True, False)])
@pytest.mark.parametrize("n", [8 * 1000 + 5, 16])
def test_sgd_step(dev, gdt, use_mom, do_sr, n):
    g = torch.Generator().manual_seed(n)
    w = (torch.rand(n, generator=g) - 0.5).to(torch.bfloat16)
    grad = (torch.randn(n, generator=g) * 0.05).to(gdt)
    m = torch.randn(n, generator=g) * 0.01
    wd_, gd_, md_ = w.to(dev), grad.to(dev), m.to(dev)
    _lib.call("haste_sgd_sr_step", wd_.data_ptr(), gd_.data_ptr(), _C.dtype_code(gdt),
              md_.data_ptr() if use_mom else None, n, 0.05, 1e-4, 0.9, int(use_mom), int(do_sr),
              2**33 + 42, 0, _C.stream_of(wd_))
    if gdt == torch.float32:
        g_np = grad.numpy()
    elif gdt == torch.bfloat16:
        g_np = bits(grad)
    else:
        g_np = grad.numpy()
    ref_w, ref_m = oracle.sgd_sr_step(bits(w), g_np, m.numpy() if use_mom else None, 0.05, 1e-4,
                                      0.9, use_mom, do_sr, 2**33 + 42)
    assert np.array_equal(bits(wd_), ref_w)
    if use_mom:
        assert np.array_equal(md_.cpu().numpy().view(np.uint32), ref_m.view(np.uint32))


def test_sgd_step_config1_size(dev):
    """Full BASELINE config-1 weight tensor (131073 x 128), fp32 grad, seed 42."""
    n = 131073 * 128
    g = torch.Generator().manual_seed(0)
    w = ((torch.rand(n, generator=g) * 2 - 1) / math.sqrt(128)).to(torch.bfloat16)
    grad = torch.randn(n, generator=g) * 1e-2
    wd_, gd_ = w.to(dev), grad.to(dev)
    _lib.call("haste_sgd_sr_step", wd_.data_ptr(), gd_.data_ptr(), _lib.DTYPE_F32, None, n, 0.05,
              1e-4, 0.0, 0, 1, 42, 0, _C.stream_of(wd_))
    ref_w, _ = oracle.sgd_sr_step(bits(w), grad.numpy(), None, 0.05, 1e-4, 0.0, False, True, 42)
    assert np.array_equal(bits(wd_), ref_w)


def test_sgd_update_api(dev):
    from haste_amd.sr_triton import sgd_update
    w = (torch.rand(4096) - 0.5).to(torch.bfloat16)
    grad = torch.randn(4096) * 0.01
    buf = torch.zeros(4096)
    wd_ = w.to(dev)
    sgd_update(wd_, grad.to(dev), buf.to(dev), 0.05, 1e-4, 0.0, True, True, 7)
    ref_w, _ = oracle.sgd_sr_step(bits(w), grad.numpy(), None, 0.05, 1e-4, 0.0, False, True, 7)
    assert np.array_equal(bits(wd_), ref_w)


@pytest.mark.parametrize("gdt", GRAD_DTYPES)
@pytest.mark.parametrize("use_mom,do_sr", [(False, True), (True, True), (True, False)])
@pytest.mark.parametrize("n", [8 * 1000 + 5, 16])
def test_sgd_step_f16_weights(dev, gdt, use_mom, do_sr, n):
    """fp16 weights (haste_sgd_sr_step_f16): bit-identical to the oracle's step
    on fp16 weights, which is pinned on the CPU to the bf16-weight step followed
    by numpy's fp16 conversion."""
    g = torch.Generator().manual_seed(n + 1)
    w = ((torch.rand(n, generator=g) - 0.5) * 4).to(torch.float16)
    grad = (torch.randn(n, generator=g) * 0.05).to(gdt)
    m = torch.randn(n, generator=g) * 0.01
    wd_, gd_, md_ = w.to(dev), grad.to(dev), m.to(dev)
    _lib.call("haste_sgd_sr_step_f16", wd_.data_ptr(), gd_.data_ptr(), _C.dtype_code(gdt),
              md_.data_ptr() if use_mom else None, n, 0.05, 1e-4, 0.9, int(use_mom), int(do_sr),
              2**33 + 43, 0, _C.stream_of(wd_))
    g_np = bits(grad) if gdt == torch.bfloat16 else grad.numpy()
    ref_w, ref_m = oracle.sgd_sr_step_f16w(w.numpy(), g_np, m.numpy() if use_mom else None, 0.05,
                                           1e-4, 0.9, use_mom, do_sr, 2**33 + 43)
    assert np.array_equal(wd_.cpu().numpy().view(np.uint16), ref_w.view(np.uint16))
    if use_mom:
        assert np.array_equal(md_.cpu().numpy().view(np.uint32), ref_m.view(np.uint32))


def test_srsgd_f16_and_bf16_params(dev):
    """SRSgd over an fp16 and a bf16 parameter (the reference sends both to
    sgd_update): each matches the oracle with the step's seed, offsets from 0."""
    from haste_amd.optim_sr import SRSgd
    g = torch.Generator().manual_seed(3)
    p16 = torch.nn.Parameter((torch.rand(1000, generator=g) - 0.5).to(torch.float16).to(dev))
    pbf = torch.nn.Parameter((torch.rand(777, generator=g) - 0.5).to(torch.bfloat16).to(dev))
    w16, wbf = p16.detach().cpu().clone(), pbf.detach().cpu().clone()
    g16 = (torch.randn(1000, generator=g) * 0.05).to(torch.float16)
    gbf = (torch.randn(777, generator=g) * 0.05).to(torch.bfloat16)
    p16.grad, pbf.grad = g16.to(dev), gbf.to(dev)
    opt = SRSgd([p16, pbf], lr=0.05, weight_decay=1e-4, momentum=0.9, seed=19)
    opt.step()
    m16 = np.zeros(1000, np.float32)
    mbf = np.zeros(777, np.float32)
    ref16, _ = oracle.sgd_sr_step_f16w(w16.numpy(), g16.numpy(), m16, 0.05, 1e-4, 0.9, True,
                                       True, 19)
    refbf, _ = oracle.sgd_sr_step(bits(wbf), bits(gbf), mbf, 0.05, 1e-4, 0.9, True, True, 19)
    assert np.array_equal(p16.detach().cpu().numpy().view(np.uint16), ref16.view(np.uint16))
    assert np.array_equal(bits(pbf.detach()), refbf)


@pytest.mark.parametrize("use_mom", [False, True])
def test_sgd_multi_matches_per_tensor_oracle(dev, use_mom):
    """One launch over tensors of mixed sizes (tails, an unaligned view, an empty one)
    with their own offset bases equals one oracle call per tensor."""
    sizes = [131073 * 8 + 3, 131073, 5, 0, 4096, 17]
    offs = [0, 0, 7, 0, 2**32 - 2, 123]
    g = torch.Generator().manual_seed(11)
    ws, gs, ms, views = [], [], [], []
    for i, n in enumerate(sizes):
        w = (torch.rand(n + 1, generator=g) - 0.5).to(torch.bfloat16)
        gr = torch.randn(n + 1, generator=g) * 0.05
        m = torch.randn(n + 1, generator=g) * 0.01
        ws.append(w), gs.append(gr), ms.append(m)
        sl = slice(1, n + 1) if i == 1 else slice(0, n)  # tensor 1 is a 2-byte-offset view
        views.append((w.to(dev)[sl], gr.to(dev)[sl], m.to(dev)[sl], sl))
    arr = (_lib.SgdTensor * len(sizes))(*[
        _lib.SgdTensor(w.data_ptr(), gr.data_ptr(), m.data_ptr() if use_mom else None, n, off)
        for (w, gr, m, _), n, off in zip(views, sizes, offs)])
    _lib.call("haste_sgd_sr_step_multi", arr, len(sizes), _lib.DTYPE_F32, 0.05, 1e-4, 0.9,
              int(use_mom), 1, 2**32 + 5, _C.stream_of(views[0][0]))
    for (w, gr, m, sl), n, off, w0, g0, m0 in zip(views, sizes, offs, ws, gs, ms):
        ref_w, ref_m = oracle.sgd_sr_step(bits(w0[sl]), g0[sl].numpy(),
                                          m0[sl].numpy() if use_mom else None, 0.05, 1e-4, 0.9,
                                          use_mom, True, 2**32 + 5, off)
        assert np.array_equal(bits(w), ref_w), n
        if use_mom:
            assert np.array_equal(m.cpu().numpy().view(np.uint32), ref_m.view(np.uint32)), n


@pytest.mark.parametrize("B,D,ldt", [(512, 768, 512), (50, 300, 64), (1, 7, 8), (130, 64, 192),
                                     (33, 65, 40), (100, 200, 104), (64, 4096, 64)])
def test_transpose_features(dev, B, D, ldt):
    x = torch.randn(B, D + 3).to(torch.bfloat16)
    xd = x.to(dev)[:, :D] if D % 8 else x.to(dev)[:, :D].contiguous()
    out = torch.full((D, ldt), 7.0, dtype=torch.bfloat16, device=dev)
    _lib.call("haste_transpose_features", xd.data_ptr(), xd.stride(0), out.data_ptr(), ldt, B, D,
              _C.stream_of(xd))
    o = out.cpu()
    assert torch.equal(o[:, :B], x[:, :D].t())
    assert torch.count_nonzero(o[:, B:].float()) == 0


REWIRE_CASES = [
    # O, F, G, D, prune, k/thr, regrow, init
    (4096, 32, 32, 768, "fraction", 4, "random", "zero"),
    (131073 // 16, 128, 64, 768, "fraction", 19, "random", "zero"),
    (10000, 64, 64, 768, "fraction", 9, "unused", "zero"),
    (3000, 64, 16, 100, "threshold", 0.05, "random", "random"),
    (2000, 256, 128, 4096, "fraction", 38, "unused", "random"),
    (777, 16, 32, 40, "fraction", 8, "unused", "random"),
    (20000, 128, 128, 768, "fraction", 19, "unused", "zero"),   # config 4's rewire shape
    # rows of 26 bytes: groups start off 16-byte boundaries and W ends mid-piece
    (1001, 13, 7, 50, "fraction", 3, "unused", "random"),
    (257, 1, 4, 9, "fraction", 1, "unused", "zero"),
    (300, 200, 300, 1000, "fraction", 30, "unused", "zero"),    # one group in 5 row chunks
    # more groups than resident workgroups: each workgroup takes several in turn
    (120000, 32, 16, 300, "threshold", 0.03, "random", "random"),
    (150000, 64, 32, 768, "fraction", 9, "unused", "random"),
]


# every case with W at the start of its allocation, and the small ones (O <= 2000)
# with W one element into it
REWIRE_PARAMS = ([c + (0,) for c in REWIRE_CASES]
                 + [c + (1,) for c in REWIRE_CASES if c[0] <= 2000])


@pytest.mark.parametrize("O,F,G,D,prune,kt,regrow,init,woff", REWIRE_PARAMS)
def test_rewire(dev, O, F, G, D, prune, kt, regrow, init, woff):
    """woff=1: W starts one element into its allocation (2 bytes off a 16-byte
    boundary), so no group is written back as whole 16-byte pieces."""
    rng = np.random.default_rng(O)
    bound = 1.0 / math.sqrt(F)
    w = oracle.f32_to_bf16_bits(rng.uniform(-bound, bound, (O, F)).astype(np.float32))
    Gc = (O + G - 1) // G
    idx = rng.integers(0, D, (Gc, F)).astype(np.int32)
    pm = oracle.PRUNE_FRACTION if prune == "fraction" else oracle.PRUNE_THRESHOLD
    k = kt if prune == "fraction" else 0
    thr = float(kt) if prune == "threshold" else 0.0
    rm = oracle.REGROW_UNUSED if regrow == "unused" else oracle.REGROW_RANDOM
    im = oracle.INIT_RANDOM if init == "random" else oracle.INIT_ZERO
    seed = 0x1234ABCD5678 + O
    ref_w, ref_idx, ref_n, ref_s, _ = oracle.rewire(w, idx, G, D, prune_mode=pm, threshold=thr, k=k,
                                                    regrow_mode=rm, init_mode=im, bound=bound, seed=seed)
    buf = torch.full((O * F + 2 * woff,), 7, dtype=torch.int16)
    buf[woff:woff + O * F] = torch.from_numpy(w.view(np.int16).reshape(-1))
    bufd = buf.to(dev)
    Wd = bufd[woff:woff + O * F].view(torch.bfloat16).view(O, F)
    idxd = torch.from_numpy(idx).to(dev)
    scores = torch.empty(Gc, F, device=dev)
    cnt = torch.zeros(1, dtype=torch.int32, device=dev)
    _lib.call("haste_rewire", Wd.data_ptr(), _lib.DTYPE_BF16, idxd.data_ptr(), scores.data_ptr(),
              cnt.data_ptr(), O, F, G, D, pm, thr, k, rm, im, bound, seed, _C.stream_of(Wd))
    assert np.array_equal(scores.cpu().numpy().view(np.uint32), ref_s.view(np.uint32))
    assert np.array_equal(idxd.cpu().numpy(), ref_idx)
    assert np.array_equal(bits(Wd), ref_w)
    b = bufd.cpu()   # the elements either side of W are untouched
    assert torch.all(b[:woff] == 7) and torch.all(b[woff + O * F:] == 7)
    assert int(cnt.item()) == ref_n


# ---- the application's variant (GroupFixedFanInReal.rewire) against the oracle ----
APP_CASES = [
    # O, F, G, D, score, grad, prune, regrow, init
    (1000, 64, 32, 300, "mean", None, "fraction", "random", "zero"),
    (1000, 64, 32, 300, "max", None, "fraction", "unused", "random"),
    (777, 128, 64, 768, "mean", "bf16", "fraction", "random", "random"),
    (777, 128, 64, 768, "max", "f32", "threshold", "random", "zero"),
    (300, 16, 16, 50, "max", "bf16", "fraction", "unused", "zero"),
    (513, 256, 128, 1000, "mean", "f32", "fraction", "random", "zero"),
]


@pytest.mark.parametrize("O,F,G,D,score,gk,prune,regrow,init", APP_CASES)
def test_app_rewire(dev, O, F, G, D, score, gk, prune, regrow, init):
    from haste_amd.rewire import GroupFixedFanInReal
    torch.manual_seed(O + F)
    layer = GroupFixedFanInReal(D, O, F, group_size=G, prune_mode=prune,
                                rewire_threshold=0.0 if prune == "threshold" else None,
                                rewire_fraction=0.15 if prune == "fraction" else None,
                                init_mode=init, score_mode=score, regrow_mode=regrow,
                                fp32_grads=gk == "f32", dtype=torch.bfloat16)
    w = bits(layer.weights)
    idx = layer.group_locations.numpy().copy()
    sm = oracle.SCORE_MAX if score == "max" else oracle.SCORE_MEAN
    g_np = None
    if gk is not None:
        gt = torch.randn(O, F, generator=torch.Generator().manual_seed(5)) * 1e-2
        gt = gt.to(torch.bfloat16) if gk == "bf16" else gt
        g_np = bits(gt) if gk == "bf16" else gt.numpy()
    if prune == "threshold":  # prune about half: the median score
        layer.rewire_threshold = float(np.median(oracle.rewire_scores_ex(w, G, sm, g_np)))
    layer = layer.to(dev)
    if gk is not None:
        layer.use_grad = True
        layer.weights.grad = gt.to(dev)
    Gc = (O + G - 1) // G
    seed = 0xABCDEF + O
    pm = oracle.PRUNE_THRESHOLD if prune == "threshold" else oracle.PRUNE_GLOBAL_FRACTION
    k = 0 if prune == "threshold" else int(Gc * F * 0.15)
    ref_w, ref_idx, ref_n, _, _ = oracle.rewire_ex(
        w, idx, G, D, prune_mode=pm, score_mode=sm, grad=g_np,
        threshold=getattr(layer, "rewire_threshold", 0.0), k=k,
        regrow_mode=oracle.REGROW_UNUSED if regrow == "unused" else oracle.REGROW_RANDOM,
        init_mode=oracle.INIT_RANDOM if init == "random" else oracle.INIT_ZERO,
        bound=1.0 / math.sqrt(F), seed=seed)
    layer.rewire(seed=seed)
    torch.cuda.synchronize()
    assert layer.pruned_total == ref_n
    assert np.array_equal(layer.group_locations.cpu().numpy(), ref_idx)
    assert np.array_equal(bits(layer.weights), ref_w)
    if prune == "fraction":
        assert ref_n == k


@pytest.mark.parametrize("n,seed", [(1, 42), (64, 42), (1000, 2**32 + 7), (262144 + 13, 123)])
def test_sr_words_fold(dev, n, seed):
    """haste_sr_words_fold draws exactly the tl.randint words of the SR kernels:
    the XOR of each 64 consecutive words, bit-exact against the oracle's randint."""
    nf = (n + 63) // 64
    fold = torch.zeros(nf, dtype=torch.int32, device=dev)
    _lib.call("haste_sr_words_fold", fold.data_ptr(), n, seed, _C.stream_of(fold))
    w = np.zeros(nf * 64, dtype=np.uint32)
    w[:n] = oracle.randint(seed, 0, n)
    exp = np.bitwise_xor.reduce(w.reshape(nf, 64), axis=1)
    assert np.array_equal(fold.cpu().numpy().view(np.uint32), exp)
