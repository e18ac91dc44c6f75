"""The entry points inside captured HIP graphs (the bench replays them that way): each kernel
family is captured once, replayed several times with eager work and synchronizations between
the replays, and every replay's output must equal the eager call's bit for bit (the kernels are
deterministic and launch nothing that a replay could repeat differently)."""
import numpy as np
import pytest

import densecore_amd as dc
from densecore_amd import synth

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q6_K = 8, 12, 14


def _replays_match(step, outputs, n_replays=3):
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.synchronize()
    want = [o.clone() for o in outputs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step()
    torch.cuda.synchronize()
    for r in range(n_replays):
        for o in outputs:
            o.fill_(float("nan")) if o.dtype.is_floating_point else o.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, w in zip(outputs, want):
            assert torch.equal(o.view(torch.uint8), w.view(torch.uint8)), f"replay {r} differs"
        _ = torch.ones(1024, device=o.device).sum().item()  # eager work between replays


MUL_MAT = [
    (Q4_K, 1, 9728, 2560),   # fused decode, 5-wave launch
    (Q8_0, 1, 3072, 1024),   # fused Q8_0 decode
    (Q6_K, 1, 2560, 9728),   # quantize + Q6_K LDS decode
    (Q6_K, 1, 1024, 2560),   # fused Q6_K decode
    (Q4_K, 64, 512, 2048),   # quantize + batched MFMA kernel
    (Q8_0, 256, 512, 2048),  # quantize + prefill MFMA kernel
]


@pytest.mark.parametrize("wt,M,N,K", MUL_MAT)
def test_mul_mat_graph_replays(dev, wt, M, N, K):
    import torch
    w = torch.from_numpy(synth.normal(N * K, 5, 0.0, 0.02).reshape(N, K)).to(dev)
    wq = dc.quantize_weights(wt, w)
    x = torch.from_numpy(synth.normal(M * K, 6).reshape(M, K)).to(dev)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    ws = torch.empty(max(dc.mul_mat_workspace_size(wt, M, K), 256), dtype=torch.uint8, device=dev)
    _replays_match(lambda: dc.mul_mat(wt, wq, N, K, x, y=y, workspace=ws,
                                      stream=torch.cuda.current_stream().cuda_stream), [y])


def test_gate_up_graph_replays(dev):
    import torch
    N, K = 9728, 2560
    wg = dc.quantize_weights(Q4_K, torch.from_numpy(synth.normal(N * K, 7, 0.0, 0.02).reshape(N, K)).to(dev))
    wu = dc.quantize_weights(Q4_K, torch.from_numpy(synth.normal(N * K, 8, 0.0, 0.02).reshape(N, K)).to(dev))
    x = torch.from_numpy(synth.normal(K, 9).reshape(1, K)).to(dev)
    y = torch.empty((1, N), dtype=torch.float32, device=dev)
    ws = torch.empty(max(dc.ffn_gate_up_workspace_size(Q4_K, 1, N, K), 256), dtype=torch.uint8, device=dev)
    _replays_match(lambda: dc.ffn_gate_up(Q4_K, wg, wu, N, K, x, y=y, workspace=ws,
                                          stream=torch.cuda.current_stream().cuda_stream), [y])


@pytest.mark.parametrize("wt,M,N,K", [(Q4_K, 1, 2560, 9728), (Q6_K, 1, 2560, 9728), (Q8_0, 64, 256, 1024)])
def test_mul_mat_add_graph_replays(dev, wt, M, N, K):
    """Projection + residual in a graph: the fused store epilogue and the add kernel after."""
    import torch
    w = torch.from_numpy(synth.normal(N * K, 14, 0.0, 0.02).reshape(N, K)).to(dev)
    wq = dc.quantize_weights(wt, w)
    x = torch.from_numpy(synth.normal(M * K, 15).reshape(M, K)).to(dev)
    r = torch.from_numpy(synth.normal(M * N, 16).reshape(M, N)).to(dev)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    ws = torch.empty(dc.mul_mat_add_workspace_size(wt, M, N, K), dtype=torch.uint8, device=dev)
    _replays_match(lambda: dc.mul_mat_add(wt, wq, N, K, x, r, y=y, workspace=ws,
                                          stream=torch.cuda.current_stream().cuda_stream), [y])


@pytest.mark.parametrize("ct,n,n_past", [(Q8_0, 1, 4095), (1, 1, 1000), (Q8_0, 9, 300), (Q8_0, 64, 100)])
def test_kv_attention_and_write_graph_replays(dev, ct, n, n_past):
    """Decode (key splits + combine) and a small prefill; the write is captured too (it writes
    the same bytes on every replay)."""
    import torch
    n_head, n_kv, hd, n_layer = 32, 8, 128, 2
    nb = (n_past + n + 15) // 16 + 1
    cache = dc.PagedKVCache(ct, nb, n_layer, n_kv, hd, device=dev)
    table = torch.arange(nb, dtype=torch.int32, device=dev).flip(0).contiguous()
    hist = torch.from_numpy(synth.normal(n_past * n_kv * hd, 10).reshape(n_past, -1)).to(dev)
    cache.write("k", 1, table, 0, hist)
    cache.write("v", 1, table, 0, hist.roll(1, 1).contiguous())
    q = torch.from_numpy(synth.normal(n * n_head * hd, 11).reshape(n, -1)).to(dev)
    kc = torch.from_numpy(synth.normal(n * n_kv * hd, 12).reshape(n, -1)).to(dev)
    vc = torch.from_numpy(synth.normal(n * n_kv * hd, 13).reshape(n, -1)).to(dev)
    out = torch.empty_like(q)
    need = dc.kv_attention_workspace_size(n_head, n_kv, hd, n, n_past)
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)

    def step():
        st = torch.cuda.current_stream().cuda_stream
        cache.attention(1, table, q, kc, vc, n_past, 0.088, out=out, workspace=ws, stream=st)
        cache.write("k", 1, table, n_past, kc, stream=st)
    _replays_match(step, [out])
    slot = dc.kv_slot_bytes(ct, n_kv * hd)
    assert np.isfinite(out.cpu().numpy()).all() and slot > 0
