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


def test_training_step_graph_replays_match_eager(dev):
    """A whole float32 training step -- the trainable forward and its backward
    (torch.autograd.grad with the output cotangent given, so that no torch
    reduction enters the graph) -- captured once and replayed on three input
    sets; every replay's output, final state and seven gradients equal the eager
    step's bit for bit."""
    B, T, H, D = 2, 512, 3, 128
    scale = D ** -0.5
    gen = torch.Generator(device=dev).manual_seed(11)
    f = torch.nn.functional
    sets = []
    for _ in range(3):
        r = lambda: torch.randn((B, T, H, D), generator=gen, device=dev)
        xs = [f.normalize(r(), dim=-1), f.normalize(r(), dim=-1), r(), torch.sigmoid(r()),
              torch.sigmoid(r()), -f.softplus(r())]
        h0 = 0.1 * torch.randn((B, H, D, D), generator=gen, device=dev)
        sets.append((xs, h0, r()))

    def step(xs, h0, do):
        out, hf = gp().gdn2_pallas_forward_trainable(*xs, scale, h0=h0)
        grads = torch.autograd.grad(out, list(xs) + [h0], grad_outputs=do)
        return out, hf, grads

    eager = []
    for xs, h0, do in sets:
        leaves = [x.clone().requires_grad_(True) for x in xs]
        h0l = h0.clone().requires_grad_(True)
        out, hf, grads = step(leaves, h0l, do)
        eager.append([out.detach().clone(), hf.detach().clone()] + [x.clone() for x in grads])
    s_xs = [x.clone().requires_grad_(True) for x in sets[0][0]]
    s_h0 = sets[0][1].clone().requires_grad_(True)
    s_do = sets[0][2].clone()
    g, res = _capture(lambda: step(s_xs, s_h0, s_do))
    out, hf, grads = res
    for rep in range(2):
        for i, (xs, h0, do) in enumerate(sets):
            with torch.no_grad():
                for s_, x in zip(s_xs, xs):
                    s_.copy_(x)
                s_h0.copy_(h0)
                s_do.copy_(do)
            g.replay()
            torch.cuda.synchronize()
            junk = torch.randn(4096, device=dev).cumsum(0)   # eager work between replays
            assert torch.isfinite(junk).all()
            got = [out, hf] + list(grads)
            for j, (a, b) in enumerate(zip(got, eager[i])):
                assert torch.equal(a, b), (rep, i, j)
