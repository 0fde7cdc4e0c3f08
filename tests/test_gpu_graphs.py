"""The serving decode step, the fused decode layer step and the prefill (at
128- and 256-wide keys) captured in HIP graphs (torch.cuda.CUDAGraph), as a serving engine captures
its decode loop: every call launches on torch's current stream and allocates
nothing itself (outputs and workspaces come from torch, so from the graph's
pool while capturing). Each test replays the graph several times with fresh
inputs copied into its static tensors, with eager work and a synchronisation
between replays, and checks every replay bit for bit against the same call
run eagerly (the kernels are deterministic: no atomics, one writer per
output)."""
import pytest
import torch

from pseudobrain_amd import gated_deltanet as gd
from pseudobrain_amd.layer import decode_layer_step

pytestmark = pytest.mark.gpu
DEV = "cuda"
REPLAYS = 4


def capture(fn):
    """fn run twice eagerly on a side stream (the library configures its
    kernels on a first call), then captured; returns (graph, fn's outputs)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    return graph, out


def test_decode_step_replays_bit_for_bit():
    """recurrent_fwd (one token per sequence, a float32 state pool stepped in
    place through state slots) in a graph against an eager pool."""
    gen = torch.Generator().manual_seed(11)
    b, slots, hk, hv, d = 8, 12, 2, 4, 128
    idx = torch.randperm(slots, generator=gen)[:b].to(torch.int32).to(DEV)
    pool0 = (torch.randn(slots, hv, d, d, generator=gen) * 0.05).to(DEV)

    def draw(seed):
        g2 = torch.Generator().manual_seed(seed)
        q = torch.nn.functional.normalize(torch.randn(b, 1, hk, d, generator=g2), dim=-1).to(torch.bfloat16)
        k = torch.nn.functional.normalize(torch.randn(b, 1, hk, d, generator=g2), dim=-1).to(torch.bfloat16)
        v = torch.randn(b, 1, hv, d, generator=g2).to(torch.bfloat16)
        g = -torch.rand(b, 1, hv, generator=g2)
        beta = torch.rand(b, 1, hv, generator=g2)
        return [x.to(DEV) for x in (q, k, v, g, beta)]

    static = draw(0)
    pool = pool0.clone()
    with torch.no_grad():
        graph, out = capture(lambda: gd.recurrent_fwd(*static, d ** -0.5, pool, pool, idx)[0])
        pool.copy_(pool0)  # the warm-up and capture calls stepped it
        ref_pool = pool0.clone()
        for r in range(REPLAYS):
            fresh = draw(100 + r)
            for s, x in zip(static, fresh):
                s.copy_(x)
            graph.replay()
            ref_o, _ = gd.recurrent_fwd(*fresh, d ** -0.5, ref_pool, ref_pool, idx)
            torch.cuda.synchronize()
            print(f"[graph decode] replay {r}", flush=True)
            assert torch.equal(out, ref_o), r
            assert torch.equal(pool, ref_pool), r


def test_decode_layer_step_replays_bit_for_bit():
    """decode_layer_step (projection row to hs, conv tails and states updated
    in place in their pools) in a graph against eager pools."""
    gen = torch.Generator().manual_seed(12)
    b, slots, hk, hv, d, conv = 8, 10, 2, 4, 128, 4
    channels = 2 * hk * d + hv * d
    width = channels + hv * d + 2 * hv
    idx = torch.randperm(slots, generator=gen)[:b].to(torch.int32).to(DEV)
    tails0 = torch.randn(slots, conv - 1, channels, generator=gen).to(DEV)
    states0 = (torch.randn(slots, hv, d, d, generator=gen) * 0.05).to(DEV)
    weight = ((torch.rand(channels, conv, generator=gen) * 2 - 1) / 2).to(DEV)
    a_log = torch.empty(hv).uniform_(0, 16, generator=gen).log().to(DEV)
    dt_bias = (torch.randn(hv, generator=gen) - 4).to(DEV)
    o_norm = (torch.rand(d, generator=gen) + 0.5).to(DEV)

    def draw(seed):
        return torch.randn(b, width, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16).to(DEV)

    z = draw(0)
    tails, states = tails0.clone(), states0.clone()

    def step(zz, tt, ss):
        return decode_layer_step(zz, tt, weight, a_log, dt_bias, ss, o_norm, hk, d, hv, d, state_idx=idx)

    with torch.no_grad():
        graph, out = capture(lambda: step(z, tails, states))
        tails.copy_(tails0)
        states.copy_(states0)
        ref_tails, ref_states = tails0.clone(), states0.clone()
        for r in range(REPLAYS):
            fresh = draw(200 + r)
            z.copy_(fresh)
            graph.replay()
            ref = step(fresh, ref_tails, ref_states)
            torch.cuda.synchronize()
            print(f"[graph decode layer] replay {r}", flush=True)
            assert torch.equal(out, ref), r
            assert torch.equal(states, ref_states) and torch.equal(tails, ref_tails), r


def test_prefill_replays_bit_for_bit():
    """chunk_fwd (its workspace from torch, so from the graph's pool) in a
    graph against eager calls, fresh inputs each replay."""
    b, t, hk, hv, d = 2, 300, 2, 4, 128

    def draw(seed):
        gen = torch.Generator().manual_seed(seed)
        q = torch.nn.functional.normalize(torch.randn(b, t, hk, d, generator=gen), dim=-1).to(torch.bfloat16)
        k = torch.nn.functional.normalize(torch.randn(b, t, hk, d, generator=gen), dim=-1).to(torch.bfloat16)
        v = torch.randn(b, t, hv, d, generator=gen).to(torch.bfloat16)
        g = -torch.rand(b, t, hv, generator=gen) * 0.5
        beta = torch.rand(b, t, hv, generator=gen)
        h0 = torch.randn(b, hv, d, d, generator=gen) * 0.05
        return [x.to(DEV) for x in (q, k, v, g, beta, h0)]

    static = draw(0)
    with torch.no_grad():
        graph, (out, final) = capture(lambda: gd.chunk_fwd(*static[:5], d ** -0.5, static[5]))
        for r in range(REPLAYS):
            fresh = draw(300 + r)
            for s, x in zip(static, fresh):
                s.copy_(x)
            graph.replay()
            ref_o, ref_s = gd.chunk_fwd(*fresh[:5], d ** -0.5, fresh[5])
            torch.cuda.synchronize()
            print(f"[graph prefill] replay {r}", flush=True)
            assert torch.equal(out, ref_o) and torch.equal(final, ref_s), r


def test_prefill_256_wide_keys_replays_bit_for_bit():
    """chunk_fwd at K = 256 (the prep kernel, then the scan for 256-wide keys)
    in a graph against eager calls, fresh inputs each replay."""
    b, t, hk, hv, d = 1, 200, 2, 4, 256

    def draw(seed):
        gen = torch.Generator().manual_seed(seed)
        q = torch.nn.functional.normalize(torch.randn(b, t, hk, d, generator=gen), dim=-1).to(torch.bfloat16)
        k = torch.nn.functional.normalize(torch.randn(b, t, hk, d, generator=gen), dim=-1).to(torch.bfloat16)
        v = torch.randn(b, t, hv, d, generator=gen).to(torch.bfloat16)
        g = -torch.rand(b, t, hv, generator=gen) * 0.5
        beta = torch.rand(b, t, hv, generator=gen)
        h0 = torch.randn(b, hv, d, d, generator=gen) * 0.05
        return [x.to(DEV) for x in (q, k, v, g, beta, h0)]

    static = draw(0)
    with torch.no_grad():
        graph, (out, final) = capture(lambda: gd.chunk_fwd(*static[:5], d ** -0.5, static[5]))
        for r in range(REPLAYS):
            fresh = draw(400 + r)
            for s, x in zip(static, fresh):
                s.copy_(x)
            graph.replay()
            ref_o, ref_s = gd.chunk_fwd(*fresh[:5], d ** -0.5, fresh[5])
            torch.cuda.synchronize()
            print(f"[graph prefill K=256] replay {r}", flush=True)
            assert torch.equal(out, ref_o) and torch.equal(final, ref_s), r
