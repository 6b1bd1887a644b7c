"""Token embedding with the weight gradient on mg_embedding_bwd.

Reference mingru/minLM.py:92,99: `nn.Embedding(num_tokens, dim)` looked up on
the token ids. The forward is torch's gather (it also refuses ids outside the
table). The backward, dw[v] = sum of the output-gradient rows of the tokens
with id v, runs on three kernels that sum in a fixed order and never copy
anything to the host. torch's embedding backward copies a segment count to the
host, which holds the host at the end of every backward pass while the GPU
drains; the optimizer's host work then ran with the GPU idle (0.12-0.2 ms per
cfg3 step, beside the 0.12 ms of the backward's own kernels).
"""
import torch
import torch.nn.functional as F

from ._lib import check, lib, ptr, stream_of

MAX_VOCAB = 512  # mg_embedding_bwd's table limit


class EmbeddingFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ids, weight):
        ids = ids.contiguous()  # (a slice of the batch: one copy, shared by the gather and the backward)
        ctx.save_for_backward(ids)
        ctx.vd = tuple(weight.shape)
        return F.embedding(ids, weight)

    @staticmethod
    def backward(ctx, dy):
        (ids,) = ctx.saved_tensors
        V, D = ctx.vd
        dx = dy.reshape(-1, D)
        if dx.dtype != torch.float32 or dx.stride(1) != 1 or dx.stride(0) % 4 or dx.data_ptr() % 16:
            dx = dx.float().contiguous()
        flat = ids.reshape(-1)
        if not flat.is_contiguous():
            flat = flat.contiguous()
        N = flat.numel()
        dw = torch.empty(V, D, dtype=torch.float32, device=dx.device)
        L = lib()
        ws = torch.empty(L.mg_embedding_bwd_workspace_bytes(N, D, V), dtype=torch.uint8, device=dx.device)
        check(L.mg_embedding_bwd(ptr(flat), ptr(dx), dx.stride(0), N, D, V, ptr(dw), D, ptr(ws), ws.numel(),
                                 stream_of(dx)), "mg_embedding_bwd")
        return None, dw


def embedding(ids: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """F.embedding(ids, weight); the weight gradient of an fp32 table of at most
    MAX_VOCAB rows (the reference's byte vocabulary is 256) goes through
    mg_embedding_bwd, other tables through torch's backward."""
    V, D = weight.shape
    if (torch.is_grad_enabled() and weight.requires_grad and weight.is_cuda and weight.dtype == torch.float32
            and ids.dtype == torch.int64 and 1 <= V <= MAX_VOCAB and D % 4 == 0 and ids.numel() > 0
            and ids.numel() < (1 << 31)):
        return EmbeddingFn.apply(ids, weight)
    return F.embedding(ids, weight)
