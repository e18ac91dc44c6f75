"""dcq_mul_mat_noalloc: dcq_mul_mat with the library's static device scratch as its workspace.

Checked through the C ABI against dcq_mul_mat (workspace = NULL: stream-ordered scratch) on the
same inputs, over pairs of calls in a row where the second is smaller than the first, so the
second call runs over scratch that still holds the first call's activation. Both entry points
run the same kernels on the same quantized bytes, so the outputs must be equal bit for bit; a
sample of rows is also checked against the CPU oracle (quantized bytes exact, fp32 within
1e-4 * max(|y|, L1)).
"""
import numpy as np
import pytest

import densecore_amd as dc
from densecore_amd import synth

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q6_K = 8, 12, 14


def _inputs(O, wt, M, N, K, seed):
    w = synth.normal(N * K, 5100 + seed, 0.0, 0.02).reshape(N, K)
    x = synth.normal(M * K, 5200 + seed).reshape(M, K)
    return O.quantize_matrix(wt, w), x


# (type, M, N, K) pairs: the second call of each pair is smaller than the first
PAIRS = [
    ((Q8_0, 2048, 1024, 2048), (Q8_0, 40, 512, 1024)),    # prefill MFMA kernel, then the generic MMQ
    ((Q4_K, 64, 2048, 2048), (Q4_K, 16, 1024, 1024)),     # batch kernel at two sizes
    ((Q6_K, 24, 512, 2560), (Q6_K, 9, 256, 512)),          # MMQ Q6_K at two sizes
    ((Q4_K, 1, 4096, 2560), (Q4_K, 3, 512, 1024)),         # fused decode: no scratch needed
]


@pytest.mark.parametrize("first,second", PAIRS, ids=lambda c: f"t{c[0]}_M{c[1]}_N{c[2]}_K{c[3]}")
def test_noalloc_matches_mul_mat(O, dev, first, second):
    import torch
    for i, (wt, M, N, K) in enumerate((first, second)):
        print(f"noalloc case type={wt} M={M} N={N} K={K} call={i}", flush=True)
        wq, x = _inputs(O, wt, M, N, K, seed=M + N + K)
        wd = torch.from_numpy(wq).to(dev)
        xd = torch.from_numpy(x).to(dev)
        y_ref = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
        y_na = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
        dc.mul_mat(wt, wd, N, K, xd, y=y_ref)
        dc.mul_mat_noalloc(wt, wd, N, K, xd, y_na)
        torch.cuda.synchronize()
        a, b = y_na.cpu().numpy(), y_ref.cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"call {i}: differs from dcq_mul_mat"
        rows = np.unique(np.linspace(0, M - 1, min(M, 12)).astype(int))
        want, l1 = O.mul_mat(wt, wq, x[rows])
        O.assert_close(a[rows], want, l1, 1e-4, what=f"noalloc type {wt} M={M} call {i}")


def test_noalloc_rejects_products_beyond_the_scratch(dev):
    """A product whose activation workspace exceeds the static array is refused before any launch."""
    import torch
    K = 4096
    M = dc.NOALLOC_SCRATCH_BYTES // K + 8  # M*K int8 alone exceeds the array
    assert dc.mul_mat_workspace_size(Q8_0, M, K) > dc.NOALLOC_SCRATCH_BYTES
    w = torch.zeros((16, dc.row_size(Q8_0, K)), dtype=torch.uint8, device=dev)
    x = torch.zeros((M, K), dtype=torch.float32, device=dev)
    y = torch.full((M, 16), 7.0, dtype=torch.float32, device=dev)
    with pytest.raises(dc.DcqError) as ei:
        dc.mul_mat_noalloc(Q8_0, w, 16, K, x, y)
    assert ei.value.status == -11
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())  # nothing was launched
