"""GPU: the operator calls are capturable into a HIP graph, and every replay gives the eager result.

The boundary promises that every entry point only enqueues (no allocation, host sync or readback
inside), so a decode step can be captured once and replayed. Each test captures a sequence, then
replays it several times with the program's own eager work in between (which reuses the caching
allocator's blocks and the GPU's caches), and checks each replay bit for bit against the eager
outputs."""
import pytest
import torch

import synth
from conftest import pkg

pytestmark = pytest.mark.gpu


def _capture(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm-up on a side stream, as torch requires before capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = fn()
    return g, outs


def _replays_match(g, outs, eager, noise):
    for rep in range(4):
        noise(rep)
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), f"replay {rep} differs"


def test_decode_linears_replay(kernels, dev):
    """One- and multi-row decode calls (fused quant, act-quant + GEMV), the fused-SiLU arm and a
    prefill-arm call in one graph."""
    K, N, g = 4096, 1024, 128
    w, s, _ = synth.int4_weight(N, K, g, seed=1, asym=False)
    tiles, sd = kernels.repack_w4(w.to(dev)), s.to(dev)
    xs = [synth.activations(M, K, seed=M).to(dev) for M in (1, 2, 5, 16, 300)]

    def step():
        outs = [kernels.w4a8_linear(x, tiles, sd, None, g) for x in xs]
        outs.append(kernels.w4a8_linear_silu(xs[0], tiles, sd, None, g))
        return outs

    eager = step()
    torch.cuda.synchronize()
    graph, outs = _capture(step)
    scratch = [torch.empty(1 << 20, device=dev)]

    def noise(rep):
        scratch[0].normal_()
        kernels.w4a8_linear(xs[2] * (rep + 2), tiles, sd, None, g)  # eager work between replays

    _replays_match(graph, outs, eager, noise)


@pytest.mark.parametrize("T", [1, 16, 300])
def test_moe_replay(kernels, dev, T):
    """Route + align (+ the one-launch prep for small batches), both grouped GEMMs, the re-quant and
    the combine: the align's device-side ntp drives every later kernel inside the graph."""
    E, top_k, H, I, g = 32, 4, 1024, 512, 128
    w13, s13, _ = synth.int4_weight(2 * I, H, g, seed=11, asym=False, E=E)
    w2, s2, _ = synth.int4_weight(H, I, g, seed=12, asym=False, E=E)
    t13, t2 = kernels.repack_w4(w13.to(dev)), kernels.repack_w4(w2.to(dev))
    s13d, s2d = s13.to(dev), s2.to(dev)
    x = synth.activations(T, H, seed=T).to(dev)
    logits = synth.router_logits(T, E, seed=T + 1).to(dev)

    def step():
        return [kernels.w4a8_moe(x, t13, s13d, None, t2, s2d, None, logits, top_k, True)]

    eager = step()
    torch.cuda.synchronize()
    graph, outs = _capture(step)
    other = synth.router_logits(T, E, seed=99).to(dev)

    def noise(rep):
        kernels.w4a8_moe(x, t13, s13d, None, t2, s2d, None, other, top_k, True)  # a different route

    _replays_match(graph, outs, eager, noise)


def test_producer_norm_replay(kernels, dev):
    """The producer norm (residual add + quant epilogue) feeding a linear on its pair: the residual
    is restored before each replay, since the graph updates it in place."""
    N_ = pkg("layers.norm")
    K, Nout, g = 4096, 512, 128
    w, s, _ = synth.int4_weight(Nout, K, g, seed=3, asym=False)
    tiles, sd = kernels.repack_w4(w.to(dev)), s.to(dev)
    x = synth.activations(8, K, seed=4).to(dev)
    r0 = synth.activations(8, K, seed=5).to(dev)
    r = r0.clone()
    gain = (torch.randn(K, device=dev) * 0.1 + 1).to(torch.bfloat16)

    def step():
        h, q, sc = N_._rms_norm_add_quant(x, r, gain, 1e-6)
        return [h, q, sc, kernels.w4a8_linear(h, tiles, sd, None, g, x_fp8=q, act_scales=sc), r]

    eager = [t.clone() for t in step()]
    r.copy_(r0)
    torch.cuda.synchronize()
    graph, outs = _capture(step)

    def noise(rep):
        r.copy_(r0)
        N_._rms_norm(x * (rep + 1), gain, 1e-6)

    _replays_match(graph, outs, eager, noise)
