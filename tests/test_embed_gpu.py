"""Token-embedding weight gradient on mg_embedding_bwd (reference
mingru/minLM.py:92,99: nn.Embedding's backward, a scatter-add of the output
gradient rows by token id), against a float64 index_add on the host:
uniform and heavily skewed ids (one id on half the tokens: many chunks),
ragged token counts, vocabularies of 1, 7, 256 and 512 rows, repeat calls bit
for bit, ids outside the table skipped, and the autograd path against
torch's nn.Embedding backward."""
import pytest
import torch

from gruboros_amd import _lib
from gruboros_amd.embed import EmbeddingFn, embedding

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ref(ids, dx, V):
    out = torch.zeros(V, dx.shape[1], dtype=torch.float64)
    ok = (ids >= 0) & (ids < V)
    out.index_add_(0, ids[ok].cpu(), dx[ok].double().cpu())
    return out


def _call(ids, dx, V):
    L = _lib.lib()
    N, D = dx.shape
    dw = torch.full((V, D), float("nan"), dtype=torch.float32, device=DEV)
    ws = torch.empty(L.mg_embedding_bwd_workspace_bytes(N, D, V), dtype=torch.uint8, device=DEV)
    _lib.check(L.mg_embedding_bwd(_lib.ptr(ids), _lib.ptr(dx), dx.stride(0), N, D, V, _lib.ptr(dw), D,
                                  _lib.ptr(ws), ws.numel(), _lib.stream_of(dx)), "mg_embedding_bwd")
    return dw


def _check(dw, ref):
    err = (dw.double().cpu() - ref).abs().max().item()
    scale = ref.abs().max().item() + 1e-30
    assert err <= 2e-6 * scale + 1e-7, err


@pytest.mark.parametrize("N,D,V,dist", [
    (16384, 1024, 256, "uniform"),     # the cfg3 step
    (16384, 1024, 256, "skewed"),      # one id on half the tokens
    (1000, 64, 7, "uniform"),          # ragged N, small table
    (333, 8, 1, "uniform"),            # one row
    (4097, 2048, 512, "uniform"),      # the largest table, cfg5's width
    (130, 12, 256, "sparse"),          # most ids without tokens
])
def test_embedding_grad_matches_fp64(N, D, V, dist):
    g = torch.Generator(device=DEV).manual_seed(N + D + V)
    if dist == "skewed":
        ids = torch.randint(0, V, (N,), device=DEV, generator=g)
        ids[torch.rand(N, device=DEV, generator=g) < 0.5] = 32
    elif dist == "sparse":
        ids = torch.randint(0, 5, (N,), device=DEV, generator=g) * 50
    else:
        ids = torch.randint(0, V, (N,), device=DEV, generator=g)
    dx = torch.randn(N, D, device=DEV, generator=g)
    dw = _call(ids, dx, V)
    _check(dw, _ref(ids, dx, V))
    assert torch.equal(_call(ids, dx, V), dw)  # fixed summation order


def test_ids_outside_the_table_are_skipped_and_strides_honoured():
    g = torch.Generator(device=DEV).manual_seed(5)
    N, D, V = 700, 32, 20
    ids = torch.randint(-3, V + 3, (N,), device=DEV, generator=g)
    wide = torch.randn(N, D + 12, device=DEV, generator=g)
    dx = wide[:, :D]  # row stride D + 12
    dw = _call(ids, dx, V)
    _check(dw, _ref(ids, dx.contiguous(), V))


@pytest.mark.parametrize("shape", [(8, 2048), (3, 5)])
def test_autograd_path_matches_torch_embedding(shape):
    torch.manual_seed(7)
    V, D = 256, 64
    emb = torch.nn.Embedding(V, D).to(DEV)
    ids = torch.randint(0, V, shape, device=DEV)
    w = emb.weight.detach().clone().requires_grad_(True)
    y = embedding(ids, w)
    assert y.grad_fn is not None and type(y.grad_fn).__name__.startswith(EmbeddingFn.__name__)
    gy = torch.randn_like(y)
    y.backward(gy)
    emb(ids).backward(gy)
    torch.testing.assert_close(y.detach(), emb(ids).detach(), rtol=0, atol=0)
    _check(w.grad, _ref(ids.reshape(-1), gy.reshape(-1, D), V))
    # torch sums in another order: the two fp32 results differ by a few ulps of the row sums
    torch.testing.assert_close(w.grad, emb.weight.grad, rtol=1e-5, atol=2e-5)
