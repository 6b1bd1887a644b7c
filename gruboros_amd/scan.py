"""Autograd Functions over the fused gate-math + scan kernels (mg_scan_fwd/bwd).

Reference semantics: mingru/minGRU.py:45-69. Given the two halves of the
``to_hidden_and_gate`` projection, compute the minGRU hidden sequence
(`out` before ``to_out``) and ``next_prev_hidden``.
"""
import ctypes

import torch

from . import _lib
from ._lib import check, dtype_code, lib, ptr, raw_stream, require_cuda, stream_of


# Look-back workspaces, one per (device, stream, B, T, Di): initialised
# (zero-filled) once, then kept consistent by the kernels across calls, which
# on one stream run in order. Calls on different streams get different
# workspaces.
_WORKSPACES = {}
# Keys of the workspaces a scan has used since their last poll (only those can
# have set an error bit since; calls that run no scan, such as the decode
# path's one-token calls, then enqueue no poll).
_USED = set()


def _workspace(device, B, T, Di):
    key = (device.index, raw_stream(device), B, T, Di)
    _USED.add(key)
    ws = _WORKSPACES.get(key)
    if ws is None:
        L = lib()
        wsb = L.mg_scan_workspace_bytes(B, T, Di)
        ws = torch.empty(wsb, dtype=torch.uint8, device=device)
        check(L.mg_scan_workspace_init(ptr(ws), wsb, B, T, Di, stream_of(ws)), "mg_scan_workspace_init")
        _WORKSPACES[key] = ws
    return ws


def release_workspaces():
    """Free the cached look-back workspaces (they are re-made on demand)."""
    _WORKSPACES.clear()
    _USED.clear()


def check_workspaces():
    """Synchronise and read the error word of every cached look-back workspace
    (mg_scan_workspace_check); raises if a scan gave up a wait or found a bad
    header. The kernels never hang on a bad workspace: they set the error word
    and exit, and this is where the error surfaces."""
    L = lib()
    for (dev, sid, B, T, Di), ws in list(_WORKSPACES.items()):
        rc = L.mg_scan_workspace_check(ptr(ws), stream_of(ws))
        check(rc, f"scan workspace (device {dev}, B={B} T={T} Di={Di})")


# Errors of the cached workspaces, surfaced without a host synchronisation per
# step: one pinned host word per device, into which mg_scan_workspace_poll's
# kernel ORs a workspace's error bits (it writes only when one is set).
_ERR_WORDS = {}


def _err_word(index):
    w = _ERR_WORDS.get(index)
    if w is None:
        w = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        _ERR_WORDS[index] = w
    return w


def poll_workspaces(device=None):
    """Enqueue the asynchronous error poll of every cached workspace (of
    `device`, if given), each on the stream the workspace belongs to. Its
    result reaches the host once that stream has passed the poll;
    raise_pending_errors reads it there."""
    L = lib()
    for key, ws in list(_WORKSPACES.items()):
        dev, sid = key[0], key[1]
        if (device is not None and dev != device.index) or key not in _USED:
            continue
        _USED.discard(key)
        word = _err_word(dev)
        check(L.mg_scan_workspace_poll(ptr(ws), ctypes.c_void_p(word.data_ptr()), ctypes.c_void_p(sid)),
              "mg_scan_workspace_poll")


def raise_pending_errors():
    """Raise MingruHipError if an earlier poll reported a workspace error (a
    look-back wait that gave up, a corrupted or foreign workspace): the scan
    results since then are invalid. Reads the pinned words only, with no
    synchronisation. On an error it synchronises to name the workspace, drops
    every cached workspace (the next call makes fresh ones) and raises."""
    for dev, word in list(_ERR_WORDS.items()):
        bits = int(word[0])
        if bits == 0:
            continue
        word.zero_()
        try:
            check_workspaces()
        finally:
            release_workspaces()
        raise _lib.MingruHipError(f"a minGRU scan on device {dev} reported workspace error bits {bits:#x} "
                                  "(1: missing header or another shape, 2: corrupted ticket, 4: a look-back wait "
                                  "gave up); the scan results since the last clean poll are invalid")


def surface_errors(device):
    """Once per training step (the model's forward and the optimizer step call
    it): raise a pending workspace error, then poll the workspaces of `device`
    again. An error made in step k is polled at the start of step k + 1 and
    raised at the next call after the host has passed that point."""
    raise_pending_errors()
    if _WORKSPACES:
        poll_workspaces(device)


def _vec_ok(t: torch.Tensor) -> bool:
    """Last dim dense and the two outer strides multiples of 4 elements."""
    return t.stride(-1) == 1 and t.stride(0) % 4 == 0 and t.stride(1) % 4 == 0


def _prep_h0(h0, B, Di, device):
    if h0 is None:
        return None
    if h0.shape not in ((B, 1, Di), (B, Di)):
        raise ValueError(f"prev_hidden must be [B,1,Di] = [{B},1,{Di}], got {tuple(h0.shape)}")
    return h0.reshape(B, Di).to(device=device, dtype=torch.float32).contiguous()


def _launch_fwd(hidden, gate, h0, out_dtype, need_ckpt=False):
    """Runs mg_scan_fwd; returns (h, h_last, ckpt). ckpt (fp32 states every 8
    steps) is produced when asked for and h is not fp32: the backward needs
    fp32 states."""
    B, T, Di = hidden.shape
    L = lib()
    h = torch.empty(B, T, Di, dtype=out_dtype, device=hidden.device)
    h_last = torch.empty(B, 1, Di, dtype=torch.float32, device=hidden.device)
    ckpt = None
    if need_ckpt and out_dtype != torch.float32:
        ckpt = torch.empty(L.mg_scan_ckpt_elems(B, T, Di), dtype=torch.float32, device=hidden.device)
    ws = _workspace(hidden.device, B, T, Di)
    rc = L.mg_scan_fwd(dtype_code(hidden.dtype), ptr(hidden), ptr(gate), hidden.stride(0), hidden.stride(1),
                       ptr(h0), dtype_code(out_dtype), ptr(h), h.stride(0), h.stride(1), ptr(h_last), ptr(ckpt),
                       B, T, Di, ptr(ws), ws.numel(), stream_of(hidden))
    check(rc, "mg_scan_fwd")
    return h, h_last, ckpt


def _launch_fwd_residual(hidden, gate, h0, res):
    """x_out = res + scan(hidden, gate) (fp32, res's layout: [B, T, Di] with a unit inner stride),
    with the scan state kept as fp32 checkpoints for the backward. Returns (x_out, h_last, ckpt)."""
    B, T, Di = hidden.shape
    L = lib()
    x_out = torch.empty(B, T, Di, dtype=torch.float32, device=hidden.device)
    h_last = torch.empty(B, 1, Di, dtype=torch.float32, device=hidden.device)
    ckpt = torch.empty(L.mg_scan_ckpt_elems(B, T, Di), dtype=torch.float32, device=hidden.device)
    if res.stride() != x_out.stride():
        res = res.contiguous()
    ws = _workspace(hidden.device, B, T, Di)
    rc = L.mg_scan_fwd_residual(dtype_code(hidden.dtype), ptr(hidden), ptr(gate), hidden.stride(0), hidden.stride(1),
                                ptr(h0), ptr(res), ptr(x_out), x_out.stride(0), x_out.stride(1), ptr(h_last),
                                ptr(ckpt), B, T, Di, ptr(ws), ws.numel(), stream_of(hidden))
    check(rc, "mg_scan_fwd_residual")
    return x_out, h_last, ckpt


def _launch_bwd(hidden, gate, h0, h, ckpt, dh, dh_last, dhidden, dgate, want_dh0):
    """dhidden, dgate: outputs with a shared layout (their strides are passed). h may be None when
    ckpt holds the forward's fp32 state checkpoints (the states are rebuilt from them)."""
    B, T, Di = hidden.shape
    L = lib()
    dev = hidden.device
    hd = h.dtype if h is not None else torch.float32
    if dh is None:
        dh = torch.zeros(B, T, Di, dtype=hd, device=dev)
    elif dh.dtype != hd or not _vec_ok(dh):
        dh = dh.to(hd).contiguous()
    if dh_last is not None:
        dh_last = dh_last.reshape(B, Di).to(torch.float32).contiguous()
    dh0 = torch.empty(B, 1, Di, dtype=torch.float32, device=dev) if want_dh0 else None
    ws = _workspace(dev, B, T, Di)
    rc = L.mg_scan_bwd(dtype_code(hidden.dtype), ptr(hidden), ptr(gate), hidden.stride(0), hidden.stride(1),
                       ptr(h0), dtype_code(hd), ptr(h), h.stride(0) if h is not None else 0,
                       h.stride(1) if h is not None else 0, ptr(ckpt),
                       ptr(dh), dh.stride(0), dh.stride(1), ptr(dh_last), ptr(dhidden), ptr(dgate),
                       dhidden.stride(0), dhidden.stride(1), ptr(dh0), B, T, Di, ptr(ws), ws.numel(),
                       stream_of(hidden))
    check(rc, "mg_scan_bwd")
    return dh0


class GateScanPacked(torch.autograd.Function):
    """hg = [hidden | gate] as produced by ``to_hidden_and_gate`` ([B, T, 2*Di]).

    Returns (out [B, T, Di] in hg's dtype, next_prev_hidden [B, 1, Di] fp32).
    The backward writes d(hg) in one buffer, so the projection's backward
    consumes it without a concatenation.
    """

    @staticmethod
    def forward(ctx, hg, h0, out_dtype):
        ctx.set_materialize_grads(False)
        B, T, D2 = hg.shape
        Di = D2 // 2
        hidden, gate = hg[..., :Di], hg[..., Di:]
        h, h_last, ckpt = _launch_fwd(hidden, gate, h0, out_dtype or hg.dtype, need_ckpt=True)
        ctx.save_for_backward(hg, h0, h, ckpt)
        return h, h_last

    @staticmethod
    def backward(ctx, dh, dh_last):
        hg, h0, h, ckpt = ctx.saved_tensors
        B, T, D2 = hg.shape
        Di = D2 // 2
        if dh is None and dh_last is None:
            return None, None, None
        dhg = torch.empty_like(hg, memory_format=torch.contiguous_format)
        want_dh0 = h0 is not None and ctx.needs_input_grad[1]
        dh0 = _launch_bwd(hg[..., :Di], hg[..., Di:], h0, h, ckpt, dh, dh_last, dhg[..., :Di], dhg[..., Di:],
                          want_dh0)
        return dhg, (dh0.reshape(h0.shape) if want_dh0 else None), None


class GateScan(torch.autograd.Function):
    """Separate hidden and gate pre-activations ([B, T, Di] each, same strides)."""

    @staticmethod
    def forward(ctx, hidden, gate, h0):
        ctx.set_materialize_grads(False)
        h, h_last, ckpt = _launch_fwd(hidden, gate, h0, hidden.dtype, need_ckpt=True)
        ctx.save_for_backward(hidden, gate, h0, h, ckpt)
        return h, h_last

    @staticmethod
    def backward(ctx, dh, dh_last):
        hidden, gate, h0, h, ckpt = ctx.saved_tensors
        if dh is None and dh_last is None:
            return None, None, None
        # inputs are contiguous (gate_scan ensures it), so the gradients,
        # which the kernel writes with the inputs' strides, are too
        dhidden = torch.empty_like(hidden)
        dgate = torch.empty_like(gate)
        want_dh0 = h0 is not None and ctx.needs_input_grad[2]
        dh0 = _launch_bwd(hidden, gate, h0, h, ckpt, dh, dh_last, dhidden, dgate, want_dh0)
        return dhidden, dgate, (dh0.reshape(h0.shape) if want_dh0 else None)


def gate_scan(hidden, gate, prev_hidden=None):
    """minGRU gate math + scan on separate pre-activation tensors.

    hidden, gate: [B, T, Di] (fp32 or bf16, CUDA). prev_hidden: [B, 1, Di] or None.
    Returns (out [B, T, Di], next_prev_hidden [B, 1, Di] fp32).
    """
    require_cuda(hidden, gate, prev_hidden)
    if hidden.shape != gate.shape or hidden.dim() != 3:
        raise ValueError(f"hidden {tuple(hidden.shape)} and gate {tuple(gate.shape)} must both be [B,T,Di]")
    if hidden.dtype != gate.dtype:
        raise ValueError("hidden and gate must share a dtype")
    hidden, gate = hidden.contiguous(), gate.contiguous()
    B, T, Di = hidden.shape
    h0 = _prep_h0(prev_hidden, B, Di, hidden.device)
    return GateScan.apply(hidden, gate, h0)


def gate_scan_packed(hg, prev_hidden=None, out_dtype=None):
    """minGRU gate math + scan on the packed projection output hg = [hidden | gate].
    out_dtype: dtype of the hidden sequence (default hg's; float32 keeps the
    scan state unrounded for the residual stream)."""
    require_cuda(hg, prev_hidden)
    if hg.dim() != 3 or hg.shape[-1] % 2:
        raise ValueError(f"hg must be [B,T,2*Di], got {tuple(hg.shape)}")
    hg = hg.contiguous()  # the gradient buffer is written with hg's strides
    B, T, D2 = hg.shape
    h0 = _prep_h0(prev_hidden, B, D2 // 2, hg.device)
    return GateScanPacked.apply(hg, h0, out_dtype)
