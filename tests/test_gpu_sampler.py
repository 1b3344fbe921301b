"""Sampler kernels (HIP) vs the CPU oracle.

Softmax: within 1e-5 relative (fp32).  Rejection sampling: given the same fp32
probabilities and uniforms, path / accepted length / tokens are bit-exact.
"""
import numpy as np
import pytest
import torch

from nanovllm import _C
from nanovllm.layers.sampler import (RejectionSampler, Sampler, rejection_sample_chain,
                                     rejection_sample_tree, rejection_sample_tree_logits,
                                     rejection_sample_tree_logits_lazy, softmax_from_stats,
                                     softmax_stats, stats_eligible, temperature_softmax)
from nanovllm.spec.tree import chain_parents, random_tree
from oracle import sampler as osamp

V_QWEN = 151936


def softmax_rows(gen, shape, std, temp):
    return torch.softmax(torch.randn(*shape, generator=gen) * std / temp, -1)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,V", [(torch.bfloat16, V_QWEN), (torch.float32, V_QWEN),
                                     (torch.bfloat16, 1001), (torch.float32, 77)])
def test_temperature_softmax(dev, dtype, V):
    g = torch.Generator().manual_seed(V)
    N = 24
    logits = (torch.randn(N, V, generator=g) * 2).to(dtype)
    temps = torch.tensor([1.0, 0.8, 0.0, 0.6, 1.7, 0.0] * 4)
    print(f"[softmax] dtype={dtype} V={V}", flush=True)
    p = temperature_softmax(logits.to(dev), temps.to(dev)).cpu().numpy()
    ref = osamp.temperature_softmax(logits.float().numpy(), temps.numpy())
    np.testing.assert_allclose(p, ref, rtol=1e-5, atol=1e-35)
    greedy = temps.numpy() == 0
    assert np.array_equal(p[greedy], logits.float().numpy()[greedy])


@pytest.mark.gpu
@pytest.mark.parametrize("V", [151560, 155648, 126984, 128256, 131072, 131080, 151936 + 8 * 512 * 4])
def test_softmax_vocab_boundaries(dev, V):
    """bf16 rows at the edges of the register-resident kernel's size classes (38 and 32
    groups of 4 KB per 512 threads; 131,080 and 168,320 take the streaming kernel),
    with padded rows (stride > V), masked logits (-inf) and greedy rows."""
    g = torch.Generator().manual_seed(V)
    N = 6
    full = (torch.randn(N, V + 64, generator=g) * 2).to(torch.bfloat16)
    full[1, : V // 2] = float("-inf")          # first half masked
    full[3, torch.rand(V + 64, generator=g) < 0.9] = float("-inf")
    full[4, V - 1] = 40.0                      # the row max in the last group's last lane
    logits = full[:, :V]
    temps = torch.tensor([0.7, 1.0, 0.0, 1.3, 0.9, 0.0])
    print(f"[softmax] bf16 V={V} stride={full.stride(0)}", flush=True)
    dl = full.to(dev)[:, :V]
    p = temperature_softmax(dl, temps.to(dev)).cpu().numpy()
    ref = osamp.temperature_softmax(logits.float().numpy(), temps.numpy())
    np.testing.assert_allclose(p, ref, rtol=1e-5, atol=1e-35)
    greedy = temps.numpy() == 0
    assert np.array_equal(p[greedy], logits.float().numpy()[greedy])


def tree_case(dev, B, T, V, depth, seed, greedy_frac=0.0, delta=False, same_pq=False,
              ragged=False, chain=False):
    rng = np.random.default_rng(seed)
    g = torch.Generator().manual_seed(seed)
    P = softmax_rows(g, (B, T, V), 2.0, 0.8)
    Q = P.clone() if same_pq else softmax_rows(g, (B, T, V), 2.0, 0.8)
    parents = np.stack([chain_parents(T) if chain else random_tree(T, depth, rng)
                        for _ in range(B)])
    # draft tokens drawn from the draft rows of their parents (Gumbel-free inverse CDF)
    toks = np.zeros((B, T), np.int32)
    Qn = Q.numpy()
    for b in range(B):
        for i in range(1, T):
            row = Qn[b, parents[b, i]].astype(np.float64)
            toks[b, i] = min(int(np.searchsorted(np.cumsum(row), rng.random() * row.sum())), V - 1)
    U = rng.random((B, T)).astype(np.float32)
    Uf = rng.random(B).astype(np.float32)
    greedy = rng.random(B) < greedy_frac
    nn_ = rng.integers(1, T + 1, size=B).astype(np.int32) if ragged else None
    print(f"[rejection] B={B} T={T} V={V} seed={seed} delta={delta} ragged={ragged}", flush=True)
    res = rejection_sample_tree(P.to(dev), None if delta else Q.to(dev), torch.from_numpy(toks).to(dev),
                                torch.from_numpy(parents).to(dev), torch.from_numpy(U).to(dev),
                                torch.from_numpy(Uf).to(dev), torch.from_numpy(greedy).to(dev),
                                None if nn_ is None else torch.from_numpy(nn_).to(dev),
                                "delta" if delta else "stochastic")
    ref = osamp.rejection_sample_tree(P.numpy(), None if delta else Qn, toks, parents, U, Uf,
                                      greedy, nn_, delta)
    names = ("path", "accepted_len", "out_tokens", "next_token")
    for name, a, r in zip(names, res, ref):
        assert np.array_equal(a.cpu().numpy(), r), f"{name} differs"
    return [r for r in ref]


@pytest.mark.gpu
def test_hand_worked_cases(dev):
    """The committed hand-worked cases (stochastic, greedy and delta mode, V = 4): the
    kernel's integer outputs equal the hand-derived ones."""
    import json
    import os
    cases = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "sampler_hand.json")))
    for i, c in enumerate(cases):
        print(f"[hand] case {i} delta={c['delta']} greedy={c['greedy']}", flush=True)
        P = torch.tensor([c["P"]], dtype=torch.float32, device=dev)
        Q = None if c["delta"] else torch.tensor([c["Q"]], dtype=torch.float32, device=dev)
        T = P.shape[1]
        path, acc, toks, nxt = rejection_sample_tree(
            P, Q, torch.tensor([c["tokens"]], device=dev), torch.tensor([c["parents"]], device=dev),
            torch.tensor([c["U"]], device=dev), torch.tensor([c["Uf"]], device=dev),
            torch.tensor([c["greedy"]], device=dev), None, "delta" if c["delta"] else "stochastic")
        assert path[0].tolist() == c["path"] + [-1] * (T - len(c["path"])), i
        assert int(acc[0]) == c["accepted"] and int(nxt[0]) == c["next"], i
        want = [c["tokens"][j] for j in c["path"][1:]] + [c["next"]]
        assert toks[0, :len(want)].tolist() == want, i


@pytest.mark.gpu
def test_tree_small_vocab_many_cases(dev):
    for seed in range(6):
        tree_case(dev, B=16, T=16, V=50, depth=4, seed=seed, greedy_frac=0.25)


@pytest.mark.gpu
def test_tree_delta_mode(dev):
    for seed in range(3):
        tree_case(dev, B=16, T=24, V=300, depth=5, seed=100 + seed, delta=True)


@pytest.mark.gpu
@pytest.mark.parametrize("width,B", [(16, 60), (8, 60), (4, 60), (2, 60), (1, 60), (16, 300)])
def test_walk_widths_are_bit_identical(dev, width, B):
    """Walks bounded to 16, 8, 4, 2 and 1 workgroups per sequence (60 sequences fit the
    GPU at every width), and 300 sequences (too many for the grid of a multi-workgroup
    walk to fit on the GPU at once, so one workgroup each): every width gives the
    oracle's outputs, in stochastic, greedy and delta mode."""
    lib = _C.lib()
    prev = lib.nvx_rejection_walk_max_width(width)
    try:
        tree_case(dev, B=B, T=12, V=3000, depth=4, seed=B + width, greedy_frac=0.2)
        tree_case(dev, B=B, T=12, V=3000, depth=4, seed=B + width + 1, delta=True)
    finally:
        assert lib.nvx_rejection_walk_max_width(prev) == width


def walk_inputs(B, T, V, depth, seed, greedy_frac=0.25):
    """Stochastic tree-walk inputs (host tensors) and the oracle's outputs."""
    rng = np.random.default_rng(seed)
    g = torch.Generator().manual_seed(seed)
    P = softmax_rows(g, (B, T, V), 2.0, 0.8)
    Q = softmax_rows(g, (B, T, V), 2.0, 0.8)
    parents = np.stack([random_tree(T, depth, rng) for _ in range(B)])
    Qn = Q.numpy()
    toks = np.zeros((B, T), np.int32)
    for b in range(B):
        for i in range(1, T):
            row = Qn[b, parents[b, i]].astype(np.float64)
            toks[b, i] = min(int(np.searchsorted(np.cumsum(row), rng.random() * row.sum())), V - 1)
    U = rng.random((B, T)).astype(np.float32)
    Uf = rng.random(B).astype(np.float32)
    greedy = rng.random(B) < greedy_frac
    ref = osamp.rejection_sample_tree(P.numpy(), Qn, toks, parents, U, Uf, greedy)
    args = (P, Q, torch.from_numpy(toks), torch.from_numpy(parents), torch.from_numpy(U),
            torch.from_numpy(Uf), torch.from_numpy(greedy))
    return args, ref


@pytest.mark.gpu
@pytest.mark.parametrize("explicit", [False, True])
def test_concurrent_walks_on_two_streams(dev, explicit):
    """Two walks at 16 workgroups per sequence launched on two streams without a
    synchronisation between them, each with its own exchange workspace (the wrapper's
    one per stream, or two caller-owned zero-filled ones), twice in a row: all four
    results equal the oracle bit for bit.  8 sequences per walk, so both grids fit on
    the GPU together."""
    from nanovllm.layers.sampler import walk_workspace
    lib = _C.lib()
    prev = lib.nvx_rejection_walk_max_width(16)
    try:
        cases = [walk_inputs(8, 64, V_QWEN, 8, seed) for seed in (31, 32)]
        dev_args = [tuple(t.to(dev) for t in a) for a, _ in cases]
        streams = [torch.cuda.Stream(dev), torch.cuda.Stream(dev)]
        ws = [None, None]
        if explicit:
            n = lib.nvx_rejection_walk_workspace_size(8)
            ws = [torch.zeros(n, dtype=torch.uint8, device=dev) for _ in range(2)]
        torch.cuda.synchronize()
        for rep in range(2):
            print(f"[walk] two streams explicit={explicit} rep={rep}", flush=True)
            outs = [None, None]
            for i in range(2):
                with torch.cuda.stream(streams[i]):
                    outs[i] = rejection_sample_tree(*dev_args[i], workspace=ws[i])
            torch.cuda.synchronize()
            for i in range(2):
                for name, a, r in zip(("path", "accepted_len", "out_tokens", "next_token"),
                                      outs[i], cases[i][1]):
                    assert np.array_equal(a.cpu().numpy(), r), f"walk {i} rep {rep}: {name} differs"
        if not explicit:
            w = []
            for s in streams:
                with torch.cuda.stream(s):
                    w.append(walk_workspace(8, dev)[0])
            assert w[0].data_ptr() != w[1].data_ptr()
    finally:
        assert lib.nvx_rejection_walk_max_width(prev) == 16


@pytest.mark.gpu
def test_tree_ragged_and_odd_vocab(dev):
    tree_case(dev, B=12, T=20, V=1003, depth=5, seed=7, ragged=True, greedy_frac=0.3)


@pytest.mark.gpu
def test_tree_q_equals_p_accepts_all(dev):
    path, acc, _, _ = tree_case(dev, B=8, T=9, V=500, depth=8, seed=3, same_pq=True, chain=True)
    assert (acc == 8).all()


@pytest.mark.gpu
def test_tree64_full_vocab(dev):
    """Qwen3-8B verify shape at B=16: 64-node depth-8 trees over the full vocabulary."""
    _, acc, _, _ = tree_case(dev, B=16, T=64, V=V_QWEN, depth=8, seed=11, greedy_frac=0.25)
    assert acc.min() >= 0


@pytest.mark.gpu
@pytest.mark.parametrize("greedy", [False, True])
def test_chain_config1(dev, greedy):
    """B=8, k=4, V=151936, logits ~ N(0, 2) softmaxed at T=1 (and a greedy variant)."""
    B, k, V = 8, 4, V_QWEN
    g = torch.Generator().manual_seed(1)
    rng = np.random.default_rng(1)
    tl = torch.randn(B, k + 1, V, generator=g) * 2
    dl = torch.randn(B, k, V, generator=g) * 2
    temps = torch.zeros(B * (k + 1)) if greedy else torch.ones(B * (k + 1))
    P = temperature_softmax(tl.view(-1, V).to(dev), temps.to(dev)).view(B, k + 1, V)
    Q = torch.softmax(dl, -1)
    Qn = Q.numpy()
    draft = np.zeros((B, k), np.int32)
    for b in range(B):
        for i in range(k):
            c = np.cumsum(Qn[b, i].astype(np.float64))
            draft[b, i] = min(int(np.searchsorted(c, rng.random() * c[-1])), V - 1)
    U = rng.random((B, k)).astype(np.float32)
    Uf = rng.random(B).astype(np.float32)
    gflag = torch.full((B,), greedy)
    out = rejection_sample_chain(P, Q.to(dev), torch.from_numpy(draft).to(dev),
                                 torch.from_numpy(U).to(dev), torch.from_numpy(Uf).to(dev),
                                 gflag.to(dev))
    ref = osamp.rejection_sample_chain(P.cpu().numpy(), Qn, draft, U, Uf, gflag.numpy())
    for a, r in zip(out, ref):
        assert np.array_equal(a.cpu().numpy(), r)


@pytest.mark.gpu
def test_invalid_draft_tokens_are_rejected(dev):
    B, T, V = 4, 5, 64
    g = torch.Generator().manual_seed(5)
    P = torch.softmax(torch.randn(B, T, V, generator=g), -1)
    Q = torch.softmax(torch.randn(B, T, V, generator=g), -1)
    parents = np.tile(chain_parents(T), (B, 1))
    toks = np.array([[0, -1, 3, 4, 5], [0, V, 1, 2, 3], [0, 1, 2, 3, 4], [0, 99999, -7, 1, 2]],
                    np.int32)
    U = np.zeros((B, T), np.float32)
    Uf = np.full(B, 0.5, np.float32)
    res = rejection_sample_tree(P.to(dev), Q.to(dev), torch.from_numpy(toks).to(dev),
                                torch.from_numpy(parents).to(dev), torch.from_numpy(U).to(dev),
                                torch.from_numpy(Uf).to(dev))
    ref = osamp.rejection_sample_tree(P.numpy(), Q.numpy(), toks, parents, U, Uf, np.zeros(B, bool))
    for a, r in zip(res, ref):
        assert np.array_equal(a.cpu().numpy(), r)
    assert res[1].cpu().numpy()[[0, 1, 3]].tolist() == [0, 0, 0]


@pytest.mark.gpu
def test_sampler_distribution(dev):
    """Sampler()(logits, T): empirical frequencies over 200k draws match softmax(l/T)."""
    V, N = 12, 200_000
    logits = torch.linspace(-2, 1.5, V).repeat(N, 1)
    temps = torch.full((N,), 0.7)
    tok = Sampler()(logits.to(dev), temps.to(dev)).cpu().numpy()
    p = torch.softmax(logits[0] / 0.7, -1).numpy()
    counts = np.bincount(tok, minlength=V)
    chi2 = ((counts - N * p) ** 2 / (N * p)).sum()
    assert chi2 < 40.0, chi2  # 11 dof: p(chi2 > 40) ~ 3e-5
    tg = Sampler()(logits[:8].to(dev), torch.zeros(8).to(dev)).cpu().numpy()
    assert (tg == V - 1).all()


def check_lazy(ld, rtd, stats, args, greedy, Qn, toks, parents, U, Uf, delta):
    """The walk with lazy statistics against the oracle: it must visit exactly the
    accepted path of every sampled sequence (and no row of a greedy one), its statistics
    must match float64 (1e-5 relative), and its outputs must equal the oracle's walk on
    the probabilities softmax_from_stats rebuilds from those statistics (bit-exact).
    stats: any statistics for the rows it does not visit."""
    BT, V = ld.shape
    B = len(greedy)
    T = BT // B
    so_d = torch.full((BT, 2), float("nan"), device=ld.device)
    lazy = rejection_sample_tree_logits_lazy(ld, rtd, *args, stats_out=so_d)
    path, acc = lazy[0].cpu().numpy(), lazy[1].cpu().numpy()
    so = so_d.cpu().numpy()
    visited = ~np.isnan(so[:, 0])
    want = np.zeros(BT, bool)
    for b in range(B):
        if not greedy[b]:
            want[b * T + path[b, :acc[b] + 1]] = True
    assert np.array_equal(visited, want), "lazy walk visited other rows than its paths"
    x = ld[torch.from_numpy(np.nonzero(visited)[0]).to(ld.device)].float().cpu().numpy()
    x = x.astype(np.float64)
    a = 1.4426950408889634 / rtd.cpu().numpy()[visited].astype(np.float64)
    M = x.max(1) * a
    S = np.exp2(x * a[:, None] - M[:, None]).sum(1)
    np.testing.assert_allclose(so[visited, 0], M, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(so[visited, 1], 1.0 / S, rtol=1e-5)
    st = stats.clone()
    vis_d = torch.from_numpy(visited).to(ld.device)
    st[vis_d] = so_d[vis_d]
    P = softmax_from_stats(ld, rtd, st).cpu().numpy().reshape(B, T, V)
    ref = osamp.rejection_sample_tree(P, None if delta else Qn, toks, parents, U, Uf, greedy, None,
                                      delta)
    for name, a_, r in zip(("path", "accepted_len", "out_tokens", "next_token"), lazy[:4], ref):
        assert np.array_equal(a_.cpu().numpy(), r), f"{name}: lazy walk != oracle"
    return lazy


def fused_case(dev, B, T, V, depth, seed, dtype=torch.bfloat16, delta=False, greedy_frac=0.0,
               temp=0.8):
    """Fused sampler (softmax_stats + rejection_sample_tree_logits) against the walk on
    the probabilities softmax_from_stats materialises from the same statistics, on the
    GPU and in the oracle: bit-exact integer outputs.  Those probabilities match
    temperature_softmax within 1e-5.  Draft rows are close to the target rows, so walks
    go deep and read many rows."""
    rng = np.random.default_rng(seed)
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randn(B * T, V, generator=g) * 2).to(dtype)
    greedy = rng.random(B) < greedy_frac
    temps = torch.where(torch.from_numpy(greedy), torch.tensor(0.0), torch.tensor(temp))
    row_temps = temps.repeat_interleave(T)
    Q = torch.softmax((logits.float() + 0.3 * torch.randn(B * T, V, generator=g)) / temp, -1).view(B, T, V)
    parents = np.stack([random_tree(T, depth, rng) for _ in range(B)])
    toks = np.zeros((B, T), np.int32)
    Qn = Q.numpy()
    for b in range(B):
        for i in range(1, T):
            row = Qn[b, parents[b, i]].astype(np.float64)
            toks[b, i] = min(int(np.searchsorted(np.cumsum(row), rng.random() * row.sum())), V - 1)
    U = torch.from_numpy(rng.random((B, T)).astype(np.float32))
    Uf = torch.from_numpy(rng.random(B).astype(np.float32))
    mode = "delta" if delta else "stochastic"
    print(f"[fused] B={B} T={T} V={V} dtype={dtype} mode={mode} seed={seed}", flush=True)
    ld, rtd = logits.to(dev), row_temps.to(dev)
    assert stats_eligible(ld)
    args = (None if delta else Q.to(dev), torch.from_numpy(toks).to(dev),
            torch.from_numpy(parents).to(dev), U.to(dev), Uf.to(dev),
            torch.from_numpy(greedy).to(dev), None, mode)
    stats = softmax_stats(ld, rtd)
    fused = rejection_sample_tree_logits(ld, rtd, stats, *args)
    P = softmax_from_stats(ld, rtd, stats)
    np.testing.assert_allclose(P.cpu().numpy(), temperature_softmax(ld, rtd).cpu().numpy(),
                               rtol=1e-5, atol=1e-35)
    two = rejection_sample_tree(P.view(B, T, V), *args)
    ref = osamp.rejection_sample_tree(P.cpu().numpy().reshape(B, T, V), None if delta else Qn, toks,
                                      parents, U.numpy(), Uf.numpy(), greedy, None, delta)
    names = ("path", "accepted_len", "out_tokens", "next_token")
    for name, a, b_, r in zip(names, fused, two, ref):
        assert np.array_equal(a.cpu().numpy(), b_.cpu().numpy()), f"{name}: fused != walk on P"
        assert np.array_equal(a.cpu().numpy(), r), f"{name}: fused != oracle"
    # statistics against the float64 softmax (1e-5 relative)
    x = logits.float().numpy().astype(np.float64)
    live = row_temps.numpy() > 0
    a = 1.4426950408889634 / np.where(live, row_temps.numpy(), 1.0)
    M = x.max(1) * a
    S = np.exp2(x * a[:, None] - M[:, None]).sum(1)
    st = stats.cpu().numpy()
    np.testing.assert_allclose(st[live, 0], M[live], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(st[live, 1], 1.0 / S[live], rtol=1e-5)
    assert (st[~live] == 0).all()
    check_lazy(ld, rtd, stats, args, greedy, None if delta else Qn, toks, parents, U.numpy(),
               Uf.numpy(), delta)
    return fused


@pytest.mark.gpu
@pytest.mark.parametrize("V,dtype", [(V_QWEN, torch.bfloat16), (128256, torch.bfloat16),
                                     (1000, torch.bfloat16), (4096, torch.float32)])
def test_fused_sampler_matches_two_step(dev, V, dtype):
    """Both register-resident size classes (38 and 32 groups), the streaming kernel for
    bf16 and fp32; sampled and greedy sequences in one batch."""
    fused_case(dev, B=6, T=24, V=V, depth=5, seed=V % 97, dtype=dtype, greedy_frac=0.3)


@pytest.mark.gpu
def test_fused_sampler_delta_and_deep_trees(dev):
    fused_case(dev, B=4, T=64, V=V_QWEN, depth=8, seed=11, delta=True)
    acc = fused_case(dev, B=8, T=64, V=2048, depth=20, seed=12)[1]
    assert int(acc.max()) >= 3  # close draft rows: walks go several levels deep


@pytest.mark.gpu
def test_rejection_sampler_module_paths(dev):
    """RejectionSampler takes the lazy fused path for eligible logits (equal to the walk
    on softmax_from_stats of the statistics it reports; lazy=False: of softmax_stats) and
    the two-step path otherwise (equal to the walk on temperature_softmax)."""
    for V in (4096, 1001):  # 1001: not a multiple of 8, two-step path
        rng = np.random.default_rng(V)
        g = torch.Generator().manual_seed(V)
        B, T = 5, 12
        logits = (torch.randn(B * T, V, generator=g) * 2).to(torch.bfloat16).to(dev)
        Q = torch.softmax(torch.randn(B, T, V, generator=g), -1).to(dev)
        parents = torch.from_numpy(np.stack([random_tree(T, 4, rng) for _ in range(B)])).to(dev)
        toks = torch.from_numpy(rng.integers(0, V, size=(B, T)).astype(np.int32)).to(dev)
        U = torch.from_numpy(rng.random((B, T)).astype(np.float32)).to(dev)
        Uf = torch.from_numpy(rng.random(B).astype(np.float32)).to(dev)
        temps = torch.tensor([0.7, 0.0, 1.0, 1.3, 0.9], device=dev)
        assert stats_eligible(logits) == (V == 4096)
        rt = temps.repeat_interleave(T)
        so = torch.zeros(B * T, 2, device=dev)
        got = RejectionSampler()(logits, temps, Q, toks, parents, U, Uf, stats_out=so)
        if V == 4096:
            st = softmax_stats(logits, rt)
            eager = RejectionSampler(lazy=False)(logits, temps, Q, toks, parents, U, Uf)
            want = rejection_sample_tree(softmax_from_stats(logits, rt, st).view(B, T, V), Q, toks,
                                         parents, U, Uf, temps == 0)
            for a, b_ in zip(eager, want):
                assert torch.equal(a, b_)
            path, acc = got[0].cpu().numpy(), got[1].cpu().numpy()
            for b in range(B):
                if float(temps[b]) > 0:  # the lazy walk's statistics of its visited rows
                    rows = torch.from_numpy(b * T + path[b, :acc[b] + 1]).to(dev)
                    st[rows] = so[rows]
            P = softmax_from_stats(logits, rt, st).view(B, T, V)
        else:
            P = temperature_softmax(logits, rt).view(B, T, V)
        want = rejection_sample_tree(P, Q, toks, parents, U, Uf, temps == 0)
        for a, b_ in zip(got, want):
            assert torch.equal(a, b_)


@pytest.mark.gpu
@pytest.mark.parametrize("delta", [False, True])
def test_fused_sampler_verify8b_batch(dev, delta):
    """The Qwen3-8B verify step's whole batch: 64 sequences of 64-node depth-8 trees over
    the full vocabulary, bf16 logits, a quarter of the sequences greedy.  Inputs are made
    on the GPU (a generator seeded per mode); draft tokens are drawn from rows close to
    the target rows, so walks go deep.  Fused sampler, two-step walk and oracle agree
    bit for bit."""
    B, T, V, temp = 64, 64, V_QWEN, 0.8
    seed = 64 + int(delta)
    print(f"[verify8b batch] B={B} T={T} V={V} delta={delta} seed={seed}", flush=True)
    rng = np.random.default_rng(seed)
    g = torch.Generator(device=dev).manual_seed(seed)
    logits = (torch.randn(B * T, V, generator=g, device=dev) * 2).to(torch.bfloat16)
    greedy = rng.random(B) < 0.25
    temps = torch.where(torch.from_numpy(greedy), torch.tensor(0.0), torch.tensor(temp))
    row_temps = temps.repeat_interleave(T).to(dev)
    Q = torch.softmax((logits.float() + 0.3 * torch.randn(B * T, V, generator=g, device=dev))
                      / temp, -1).view(B, T, V)
    parents = np.stack([random_tree(T, 8, rng) for _ in range(B)])
    par = torch.from_numpy(parents).to(dev).long()
    rows = Q[torch.arange(B, device=dev)[:, None], par.clamp(min=0)]  # [B, T, V]: parent rows
    toks = torch.multinomial(rows.view(B * T, V), 1, generator=g).view(B, T).to(torch.int32)
    del rows
    toks[:, 0] = 0  # the root's token is not a proposal
    U = torch.from_numpy(rng.random((B, T)).astype(np.float32)).to(dev)
    Uf = torch.from_numpy(rng.random(B).astype(np.float32)).to(dev)
    mode = "delta" if delta else "stochastic"
    assert stats_eligible(logits)
    args = (None if delta else Q, toks, torch.from_numpy(parents).to(dev), U, Uf,
            torch.from_numpy(greedy).to(dev), None, mode)
    stats = softmax_stats(logits, row_temps)
    fused = rejection_sample_tree_logits(logits, row_temps, stats, *args)
    P = softmax_from_stats(logits, row_temps, stats)
    two = rejection_sample_tree(P.view(B, T, V), *args)
    ref = osamp.rejection_sample_tree(P.cpu().numpy().reshape(B, T, V),
                                      None if delta else Q.cpu().numpy(), toks.cpu().numpy(),
                                      parents, U.cpu().numpy(), Uf.cpu().numpy(), greedy, None,
                                      delta)
    names = ("path", "accepted_len", "out_tokens", "next_token")
    for name, a, b_, r in zip(names, fused, two, ref):
        assert np.array_equal(a.cpu().numpy(), b_.cpu().numpy()), f"{name}: fused != walk on P"
        assert np.array_equal(a.cpu().numpy(), r), f"{name}: fused != oracle"
    if not delta:  # sampled sequences walk several levels deep
        assert ref[1][~greedy].mean() >= 2
    del P, two
    check_lazy(logits, row_temps, stats, args, greedy, None if delta else Q.cpu().numpy(),
               toks.cpu().numpy(), parents, U.cpu().numpy(), Uf.cpu().numpy(), delta)
