"""Token-by-token generation for a bf16 minLM on the decode kernels.

Reference generate.py:184-212 processes the prompt with one parallel forward
and then calls ``model(prev_token, return_prev_hiddens=True,
prev_hiddens=hidden_states)`` once per generated token. ``Decoder`` keeps
that contract (``prefill`` then ``step``) with the per-token work on
``mg_decode_mingru`` / ``mg_decode_ff`` / ``mg_decode_head``: two launches
per layer plus one, captured once into a HIP graph (torch.cuda.CUDAGraph)
and replayed for every token. All buffers are allocated up front; a step
allocates nothing and does not synchronise with the host.

Requirements: ``compute_dtype=torch.bfloat16``, expansion 1.0 (no
``to_out``), no conv, no dropout, batch 1..8, dim and FeedForward width
multiples of 8 and at most 4096.
"""
import torch

from . import _lib
from ._lib import check, lib, ptr, stream_of
from .linear import bf16_copy

FP32_EPS = float(torch.finfo(torch.float32).eps)


class Decoder:
    def __init__(self, model, batch_size, graph=True):
        from .mingru.minGRU import minGRU

        if model.compute_dtype != torch.bfloat16:
            raise _lib.MingruHipError("Decoder needs a minLM built with compute_dtype=torch.bfloat16")
        if not 1 <= batch_size <= 8:
            raise _lib.MingruHipError(f"Decoder batch {batch_size} outside [1, 8]")
        for conv, _, gru, _, ff, dropout in model.layers:
            if conv is not None or dropout is not None or not isinstance(gru, minGRU) or \
                    gru.to_hidden_and_gate.weight.shape[0] != 2 * gru.to_hidden_and_gate.weight.shape[1]:
                raise _lib.MingruHipError("Decoder supports expansion 1.0 without conv or dropout")
        dev = model.token_emb.weight.device
        _lib.require_cuda(model.token_emb.weight)
        self.model, self.B, self.graph_enabled = model, batch_size, graph
        self.D = model.token_emb.weight.shape[1]
        self.V = model.token_emb.weight.shape[0]
        self.F = model.layers[0][4][0].weight.shape[0]
        B, D, F, V = self.B, self.D, self.F, self.V
        self.tokens = torch.zeros(B, dtype=torch.int64, device=dev)
        self.x = [torch.zeros(B, D, device=dev) for _ in range(2)]
        self.pending = torch.zeros(B, D, dtype=torch.bfloat16, device=dev)
        self.act = torch.zeros(B, F, dtype=torch.bfloat16, device=dev)
        self.logits = torch.zeros(B, V, dtype=torch.bfloat16, device=dev)
        self.state = [torch.zeros(B, D, device=dev) for _ in model.layers]
        self._graph = None
        self._weights = None

    # -- weights: the bf16 copies the training path also uses
    def _current_weights(self):
        m = self.model
        ws = []
        for _, _, gru, _, ff, _ in m.layers:
            ws += [bf16_copy(gru.to_hidden_and_gate.weight, dense=True), bf16_copy(ff[0].weight, dense=True),
                   bf16_copy(ff[0].bias, dense=True), bf16_copy(ff[2].weight, dense=True),
                   bf16_copy(ff[2].bias, dense=True)]
        ws.append(bf16_copy(m.to_logits.weight, dense=True))
        return ws

    def _launch(self, weights):
        L, m = lib(), self.model
        B, D, F, V = self.B, self.D, self.F, self.V
        st = stream_of(self.x[0])
        cur = 0
        for i, (_, norm, _, ff_norm, _, _) in enumerate(m.layers):
            whg, w1, b1, w2, b2 = weights[5 * i: 5 * i + 5]
            nxt = 1 - cur
            if i == 0:
                rc = L.mg_decode_mingru(B, D, ptr(self.tokens), ptr(m.token_emb.weight), V, None, None,
                                        ptr(self.x[nxt]), ptr(norm.weight), ptr(whg), ptr(self.state[i]), FP32_EPS,
                                        st)
            else:
                rc = L.mg_decode_mingru(B, D, None, None, 0, ptr(self.x[cur]), ptr(self.pending), ptr(self.x[nxt]),
                                        ptr(norm.weight), ptr(whg), ptr(self.state[i]), FP32_EPS, st)
            check(rc, "mg_decode_mingru")
            check(L.mg_decode_ff(B, D, F, ptr(self.x[nxt]), ptr(ff_norm.weight), ptr(w1), ptr(b1), ptr(self.act),
                                 ptr(w2), ptr(b2), ptr(self.pending), FP32_EPS, st), "mg_decode_ff")
            cur = nxt
        check(L.mg_decode_head(B, D, V, ptr(self.x[cur]), ptr(self.pending), ptr(m.norm.weight), ptr(weights[-1]),
                               ptr(self.logits), FP32_EPS, st), "mg_decode_head")

    def _capture(self, weights):
        side = torch.cuda.Stream(device=self.tokens.device)
        side.wait_stream(torch.cuda.current_stream())
        saved = [s.clone() for s in self.state]
        with torch.cuda.stream(side):
            self._launch(weights)  # warm-up launch outside the capture
        torch.cuda.current_stream().wait_stream(side)
        for s, v in zip(self.state, saved):
            s.copy_(v)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._launch(weights)
        for s, v in zip(self.state, saved):  # capture does not run the kernels, but keep the state exact
            s.copy_(v)
        self._graph, self._weights = g, weights

    # -- public API
    def set_hiddens(self, hiddens):
        """Load the per-layer states from prev_hiddens ([B, 1, D] each, as minLM returns them)."""
        for s, h in zip(self.state, hiddens):
            s.copy_(h.reshape(self.B, self.D))

    def hiddens(self):
        """The current per-layer states as prev_hiddens views ([B, 1, D] fp32)."""
        return [s.view(self.B, 1, self.D) for s in self.state]

    @torch.no_grad()
    def prefill(self, ids):
        """Parallel forward over the prompt ids [B, T] (reference generate.py:188);
        returns the logits of its last position [B, V] and sets the states."""
        logits, hiddens = self.model(ids, return_prev_hiddens=True)
        self.set_hiddens(hiddens)
        return logits[:, -1, :]

    @torch.no_grad()
    def step(self, tokens):
        """One token per batch row (tokens [B] int64, on the device) -> logits [B, V] bf16.
        The returned tensor is the decoder's buffer, overwritten by the next step."""
        self.tokens.copy_(tokens.reshape(self.B))
        weights = self._current_weights()
        if not self.graph_enabled:
            self._launch(weights)
            return self.logits
        if self._graph is None or any(a is not b for a, b in zip(weights, self._weights)):
            self._capture(weights)  # first step, or the weights were changed in place
        self._graph.replay()
        return self.logits
