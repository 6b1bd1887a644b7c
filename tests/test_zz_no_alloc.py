"""The allocation-free scan forward (mg_scan_fwd_noalloc), called through the
C ABI, against the workspace entry point (mg_scan_fwd) on the same inputs:
bit for bit, on two calls in a row on one device, the second with a smaller
input (the shared scratch keeps the first call's contents and must be set up
again), and with the packed projection layout and an fp32 output; inside a
captured graph; with its error word read by mg_scan_fwd_noalloc_check. Sizes
above the scratch maximum, and misaligned tensors, are refused before any
launch."""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(B, T, Di, seed, packed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    if packed:
        hg = torch.randn(B, T, 2 * Di, device=DEV, generator=g).to(torch.bfloat16)
        hidden, gate = hg[..., :Di], hg[..., Di:]
    else:
        hidden = torch.randn(B, T, Di, device=DEV, generator=g).to(torch.bfloat16)
        gate = torch.randn(B, T, Di, device=DEV, generator=g).to(torch.bfloat16)
    h0 = torch.rand(B, Di, device=DEV, generator=g) + 0.1
    return hidden, gate, h0


def _call(L, fn, hidden, gate, h0, out_dtype, ws=None):
    from gruboros_amd import _lib

    P = _lib.ptr
    B, T, Di = hidden.shape
    h = torch.full((B, T, Di), 7.0, device=DEV, dtype=out_dtype)
    h_last = torch.full((B, Di), 7.0, device=DEV)
    ckpt = torch.full((L.mg_scan_ckpt_elems(B, T, Di),), 7.0, device=DEV)
    od = _lib.dtype_code(out_dtype)
    args = [1, P(hidden), P(gate), hidden.stride(0), hidden.stride(1), P(h0), od, P(h), h.stride(0), h.stride(1),
            P(h_last), P(ckpt), B, T, Di]
    if ws is None:
        rc = L.mg_scan_fwd_noalloc(*args, _lib.stream_of(hidden))
    else:
        rc = L.mg_scan_fwd(*args, P(ws), ws.numel(), _lib.stream_of(hidden))
    assert rc == 0, L.mg_last_error()
    return h, h_last, ckpt


@pytest.mark.parametrize("packed,out_dtype", [(False, torch.bfloat16), (True, torch.float32)])
def test_noalloc_forward_matches_workspace_entry_point(packed, out_dtype):
    from gruboros_amd import _lib

    L = _lib.lib()
    # a large call then a smaller one on the same device (the scratch holds the first call's words)
    for B, T, Di, seed in ((8, 2047, 1024, 1), (3, 515, 132, 2)):
        hidden, gate, h0 = _inputs(B, T, Di, seed, packed)
        got = _call(L, "noalloc", hidden, gate, h0, out_dtype)
        ws = torch.empty(L.mg_scan_workspace_bytes(B, T, Di), dtype=torch.uint8, device=DEV)
        assert L.mg_scan_workspace_init(_lib.ptr(ws), ws.numel(), B, T, Di, _lib.stream_of(ws)) == 0
        want = _call(L, "workspace", hidden, gate, h0, out_dtype, ws)
        torch.cuda.synchronize()
        print(f"noalloc B={B} T={T} Di={Di} packed={packed} {out_dtype}", flush=True)
        for a, b in zip(got, want):
            assert torch.equal(a, b)


def test_noalloc_check_rejected_call_and_graph_capture():
    """mg_scan_fwd_noalloc_check reads the scratch's error word (0 after good
    calls); a call rejected for a misaligned tensor returns MG_ERR_ARG with
    nothing enqueued (the next check and call are clean); and the call works
    inside a captured HIP graph: each replay, with eager work and
    synchronisations between replays, equals mg_scan_fwd on the inputs the
    graph then reads."""
    from gruboros_amd import _lib

    L, P = _lib.lib(), _lib.ptr
    B, T, Di = 4, 700, 256
    hidden, gate, h0 = _inputs(B, T, Di, 5, True)
    first = _call(L, "noalloc", hidden, gate, h0, torch.float32)
    assert L.mg_scan_fwd_noalloc_check(_lib.stream_of(hidden)) == 0, L.mg_last_error()

    print("case: rejected call (misaligned h)", flush=True)
    hbuf = torch.empty(B * T * Di + 4, device=DEV)
    rc = L.mg_scan_fwd_noalloc(1, P(hidden), P(gate), hidden.stride(0), hidden.stride(1), P(h0), 0,
                               _lib.ctypes.c_void_p(hbuf.data_ptr() + 4), T * Di, Di, None, None, B, T, Di,
                               _lib.stream_of(hidden))
    assert rc == 1 and b"misaligned" in L.mg_last_error()
    assert L.mg_scan_fwd_noalloc_check(_lib.stream_of(hidden)) == 0, L.mg_last_error()
    again = _call(L, "noalloc", hidden, gate, h0, torch.float32)
    for a, b in zip(first, again):
        assert torch.equal(a, b)

    print("case: graph capture", flush=True)
    ws = torch.empty(L.mg_scan_workspace_bytes(B, T, Di), dtype=torch.uint8, device=DEV)
    assert L.mg_scan_workspace_init(P(ws), ws.numel(), B, T, Di, _lib.stream_of(ws)) == 0
    h = torch.empty(B, T, Di, device=DEV)
    h_last = torch.empty(B, Di, device=DEV)
    args = lambda: [1, P(hidden), P(gate), hidden.stride(0), hidden.stride(1), P(h0), 0, P(h), h.stride(0),  # noqa
                    h.stride(1), P(h_last), None, B, T, Di]
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        assert L.mg_scan_fwd_noalloc(*args(), _lib.stream_of(h)) == 0  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        rc = L.mg_scan_fwd_noalloc(*args(), _lib.stream_of(h))
    assert rc == 0, L.mg_last_error()
    gen = torch.Generator(device=DEV).manual_seed(11)
    for replay in range(3):
        src = torch.randn(B, T, 2 * Di, device=DEV, generator=gen).to(torch.bfloat16)
        hidden.copy_(src[..., :Di])  # hidden/gate are views of one packed buffer; refill it
        gate.copy_(src[..., Di:])
        graph.replay()
        torch.cuda.synchronize()
        want = _call(L, "workspace", hidden, gate, h0, torch.float32, ws)
        torch.cuda.synchronize()
        print(f"replay {replay}", flush=True)
        assert torch.equal(h, want[0]) and torch.equal(h_last, want[1])
        assert L.mg_scan_fwd_noalloc_check(_lib.stream_of(h)) == 0, L.mg_last_error()


def test_noalloc_refuses_sizes_above_the_scratch():
    from gruboros_amd import _lib

    L = _lib.lib()
    assert L.mg_scan_fwd_noalloc_max_bytes() == (16 << 20) + (64 << 10)
    # B16 T8192 Di2048 (cfg2) fits; twice the batch does not
    x = torch.empty(8, dtype=torch.bfloat16, device=DEV)
    P = _lib.ptr
    rc = L.mg_scan_fwd_noalloc(1, P(x), P(x), 8192 * 2048, 2048, None, 1, P(x), 8192 * 2048, 2048, None, None, 32,
                               8192, 2048, _lib.stream_of(x))
    assert rc == 1 and b"allocation-free maximum" in L.mg_last_error()
