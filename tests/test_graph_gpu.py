"""HIP graph capture of the library's calls (torch.cuda.graph): every entry point
takes caller-owned buffers and launches kernels only (no allocation, memset or
synchronisation inside), so a serving loop can capture it.  Each test captures a
call on static input buffers, replays the graph several times with new inputs
copied in and eager torch work plus a device synchronisation between the
replays, and checks every replay bit for bit against the eager call on the same
inputs (the same kernels run in both)."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def gp():
    import gdn2_package
    return gdn2_package


def _tokens(dev, gen, B, H, D, n):
    f = torch.nn.functional
    toks = []
    for _ in range(n):
        r = lambda: torch.randn((B, 1, H, D), generator=gen, device=dev)
        q, k = f.normalize(r(), dim=-1), f.normalize(r(), dim=-1)
        toks.append([x.to(torch.bfloat16) for x in (q, k, r(), torch.sigmoid(r()),
                                                     torch.sigmoid(r()))]
                    + [-f.softplus(r())])
    return toks


def _capture(fn):
    """Warm up on a side stream (default priority), then capture fn()."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        res = fn()
    return g, res


def test_decode_step_graph_replays_match_eager(dev):
    """A decode loop: one captured step (state updated in place) replayed per token."""
    B, H, D, n = 4, 6, 128, 6
    gen = torch.Generator(device=dev).manual_seed(3)
    toks = _tokens(dev, gen, B, H, D, n)
    scale = D ** -0.5
    state_e = torch.zeros((B, H, D, D), device=dev)
    outs_e = []
    for t in toks:
        o, _ = gp().gdn2_decode_step(*t, scale, state=state_e, inplace=True)
        outs_e.append(o.clone())
    static = [x.clone() for x in toks[0]]
    state_g = torch.zeros((B, H, D, D), device=dev)
    scratch = torch.zeros_like(state_g)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):   # warm-up on a side stream, on a scratch state
        gp().gdn2_decode_step(*static, scale, state=scratch, inplace=True)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2):   # captured, not run: state_g stays zero until a replay
        out_g2, _ = gp().gdn2_decode_step(*static, scale, state=state_g, inplace=True)
    state_g.zero_()
    torch.cuda.synchronize()
    for i, t in enumerate(toks):
        for s_, x in zip(static, t):
            s_.copy_(x)
        g2.replay()
        torch.cuda.synchronize()
        junk = torch.randn(4096, device=dev).cumsum(0)   # eager work between replays
        assert torch.isfinite(junk).all()
        assert torch.equal(out_g2, outs_e[i]), i
    assert torch.equal(state_g, state_e)


@pytest.mark.parametrize("chunk", [128, 64])
def test_forward_graph_replays_match_eager(dev, chunk):
    """The inference forward (bf16, D = 128; its workspace and outputs come from the
    graph's memory pool at capture) replayed on three input sets."""
    f = torch.nn.functional
    B, T, H, D = 2, 1024, 3, 128
    gen = torch.Generator(device=dev).manual_seed(7)
    sets = []
    for _ in range(3):
        r = lambda: torch.randn((B, T, H, D), generator=gen, device=dev)
        sets.append([x.to(torch.bfloat16) for x in (f.normalize(r(), dim=-1),
                                                    f.normalize(r(), dim=-1), r(),
                                                    torch.sigmoid(r()), torch.sigmoid(r()))]
                    + [-f.softplus(r())])
    scale = D ** -0.5
    eager = [[y.clone() for y in gp().gdn2_pallas_forward(*xs, scale, chunk_size=chunk)]
             for xs in sets]
    static = [x.clone() for x in sets[0]]
    g, (out, hf) = _capture(lambda: gp().gdn2_pallas_forward(*static, scale, chunk_size=chunk))
    for rep in range(2):
        for i, xs in enumerate(sets):
            for s_, x in zip(static, xs):
                s_.copy_(x)
            g.replay()
            torch.cuda.synchronize()
            junk = torch.randn(4096, device=dev).sum()
            assert torch.isfinite(junk)
            assert torch.equal(out, eager[i][0]) and torch.equal(hf, eager[i][1]), (rep, i)
