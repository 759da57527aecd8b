"""Forward + backward captured into a HIP graph (torch.cuda.graph) and replayed: every replay
equals the ordinary (eager) calls bitwise.  Covers the fp32 MFMA path, whose persistent
kernels pull tasks from device-side counters in eager mode and switch to the static
schedule under capture (also in the dS-first order), the three-plane fp32 path and the bf16
path.  Replays run in series with eager launches of the same kernel families between them
(which take queue slots), and the outputs are cleared before every replay so each replay
must write them."""
import pytest
import torch

from oracle import attention_ref as ref
from gpu_util import default_scale, to_dev


def _inputs(B, H, T, d, dtype, seed):
    q, k, v, do = ref.seeded_inputs(B, H, T, d, seed=seed)
    return tuple(to_dev(x, dtype) for x in (q, k, v, do))


def _replay_and_check(graph, outs, eager_fn, want):
    for rep in range(3):
        for t in outs:
            t.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, got, exp in zip(("o", "m", "l", "dq", "dk", "dv"), outs, want):
            assert torch.equal(got, exp), f"replay {rep}: {name} differs from eager"
        eager_fn()  # ordinary launches between replays
        torch.cuda.synchronize()


@pytest.mark.gpu
@pytest.mark.parametrize("d", [64, 128])
def test_graph_fp32_tiled(lib, d):
    B, H, T = 2, 8, 333
    scale = default_scale(d)
    q, k, v, do = _inputs(B, H, T, d, torch.float32, 11)
    r = B * H * T

    def run(o, m, l, dq, dk, dv, ws):
        lib.tiled_causal_attention_forward(q, k, v, o, B, H, T, d, scale, m, l)
        lib.tiled_causal_attention_backward(q, k, v, o, do, m, l, dq, dk, dv, ws, B, H, T, d,
                                            scale)

    mk = lambda: (torch.empty_like(q), q.new_empty(r), q.new_empty(r), torch.empty_like(q),
                  torch.empty_like(q), torch.empty_like(q), q.new_empty(r))
    want = mk()
    run(*want)
    torch.cuda.synchronize()
    scratch = mk()
    outs = mk()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run(*outs)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run(*outs)
    _replay_and_check(g, outs[:6], lambda: run(*scratch), want[:6])


@pytest.mark.gpu
def test_graph_fp32_packed_ds(lib):
    """The fp32 MFMA backward in the dS-first order (its dK/dV stage is a persistent kernel:
    queue in eager mode, static schedule under capture)."""
    B, H, T, d = 2, 4, 517, 64
    scale = default_scale(d)
    q, k, v, do = _inputs(B, H, T, d, torch.float32, 14)
    qkv = torch.stack([q, k, v], 0).permute(1, 3, 0, 2, 4).reshape(B, T, 3 * H * d).contiguous()
    r = B * H * T
    nds = lib.f32_ds_workspace_bytes(B, H, T, d) // 4

    def run(o, m, l, dqkv, ws, ds):
        lib.packed_causal_attention_forward(qkv, o, B, H, T, d, scale, m, l)
        lib.packed_causal_attention_backward_ds(qkv, o, do, m, l, dqkv, ws, ds, B, H, T, d,
                                                scale)

    mk = lambda: (torch.empty_like(q), q.new_empty(r), q.new_empty(r), torch.empty_like(qkv),
                  q.new_empty(r), q.new_empty(nds))
    want = mk()
    run(*want)
    torch.cuda.synchronize()
    scratch, outs = mk(), mk()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run(*outs)
    for rep in range(3):
        for t in outs[:5]:
            t.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for name, got, exp in zip(("o", "m", "l", "dqkv", "D"), outs[:5], want[:5]):
            assert torch.equal(got, exp), f"replay {rep}: {name} differs from eager"
        run(*scratch)
        torch.cuda.synchronize()


@pytest.mark.gpu
def test_graph_f32x3_packed(lib):
    B, H, T, d = 2, 4, 517, 64
    scale = default_scale(d)
    q, k, v, do = _inputs(B, H, T, d, torch.float32, 12)
    qkv = torch.stack([q, k, v], 0).permute(1, 3, 0, 2, 4).reshape(B, T, 3 * H * d).contiguous()
    r = B * H * T
    nbytes = lib.f32x3_workspace_bytes(B, H, T, d)

    def run(o, m, l, dqkv, ws, planes):
        lib.packed_causal_attention_forward_f32x3(qkv, o, B, H, T, d, scale, planes, m, l)
        lib.packed_causal_attention_backward_f32x3(qkv, o, do, m, l, dqkv, ws, B, H, T, d,
                                                   scale, planes, True)

    mk = lambda: (torch.empty_like(q), q.new_empty(r), q.new_empty(r), torch.empty_like(qkv),
                  q.new_empty(r), torch.empty(nbytes, dtype=torch.uint8, device=q.device))
    want = mk()
    run(*want)
    torch.cuda.synchronize()
    scratch, outs = mk(), mk()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run(*outs)
    split = lambda t: list(t.reshape(B, T, 3, H, d).permute(2, 0, 3, 1, 4))
    for rep in range(3):
        for t in outs[:5]:
            t.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for name, got, exp in zip(("o", "m", "l"), outs[:3], want[:3]):
            assert torch.equal(got, exp), f"replay {rep}: {name} differs from eager"
        for name, got, exp in zip(("dq", "dk", "dv"), split(outs[3]), split(want[3])):
            assert torch.equal(got, exp), f"replay {rep}: {name} differs from eager"
        run(*scratch)
        torch.cuda.synchronize()


@pytest.mark.gpu
def test_graph_bf16_tiled(lib):
    B, H, T, d = 2, 8, 1000, 64
    scale = default_scale(d)
    q, k, v, do = _inputs(B, H, T, d, torch.bfloat16, 13)
    r = B * H * T
    f32 = dict(dtype=torch.float32, device=q.device)

    def run(o, m, l, dq, dk, dv, ws):
        lib.tiled_causal_attention_forward(q, k, v, o, B, H, T, d, scale, m, l)
        lib.tiled_causal_attention_backward(q, k, v, o, do, m, l, dq, dk, dv, ws, B, H, T, d,
                                            scale)

    mk = lambda: (torch.empty_like(q), torch.empty(r, **f32), torch.empty(r, **f32),
                  torch.empty_like(q), torch.empty_like(q), torch.empty_like(q),
                  torch.empty(r, **f32))
    want = mk()
    run(*want)
    torch.cuda.synchronize()
    scratch, outs = mk(), mk()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run(*outs)
    _replay_and_check(g, outs[:6], lambda: run(*scratch), want[:6])
