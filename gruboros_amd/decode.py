"""Token-by-token generation for a minLM on the decode kernels (bf16, fp32 or float16 models).

Reference generate.py:184-212 processes the prompt with one parallel forward
and then calls ``model(prev_token, return_prev_hiddens=True,
prev_hiddens=hidden_states)`` once per generated token. ``Decoder`` keeps
that contract (``prefill`` then ``step``) with the per-token work on
``mg_decode_mingru`` (``mg_decode_mingru_expanded`` + ``mg_decode_to_out``
when expansion != 1) / ``mg_decode_ff`` / ``mg_decode_head``: two or three
launches per layer plus one, captured once into a HIP graph
(torch.cuda.CUDAGraph) and replayed for every token. All buffers are
allocated up front; a step allocates nothing and does not synchronise with
the host.

``minLM.forward`` also routes generate.py's own one-token calls here
(``forward_one``), so generate.py as written runs on the decode kernels.

Requirements (``unsupported_reason``): bf16 activations, i.e. a minLM built
with ``compute_dtype=torch.bfloat16`` over fp32 parameters, or one whose
parameters were cast with ``.to(torch.bfloat16)`` (generate.py:140-141); or
a model kept in fp32 (generate.py --use-f32: fp32 parameters and no
compute_dtype), which runs the *_f32 steps (fp32 weights and activations, no
rounding point); or a model cast with .to(torch.float16) (--use-f32
--use-fp16), which runs the *_f16 steps (the bf16 steps at fp16); no conv; dropout only in eval mode (where it is the
identity); batch 1..8; dim a multiple of 8 and at most 2048; the scan width
Di = dim * expansion and the FeedForward width multiples of 8 and at most
8192 (4096 for an fp32 model at batch 5-8).
"""
import weakref

import torch

from . import _lib
from ._lib import check, lib, ptr, stream_of
from .linear import bf16_copy

FP32_EPS = float(torch.finfo(torch.float32).eps)
MAX_DIM, MAX_STAGED, MAX_BATCH = 2048, 8192, 8


def _widths(model):
    """(D, Di, F, V) of a minLM."""
    gru, ff = model.layers[0][2], model.layers[0][4]
    return (model.token_emb.weight.shape[1], gru.to_hidden_and_gate.weight.shape[0] // 2, ff[0].weight.shape[0],
            model.token_emb.weight.shape[0])


def _kind(model):
    """Which decode steps serve the model: "bf16" (bf16 activations), "f32" (an fp32 model),
    "f16" (parameters cast to float16), or None."""
    cd, _ = model._dtypes()
    pd = model.token_emb.weight.dtype
    if cd == torch.bfloat16:
        return "bf16"
    if pd == torch.float16:
        return "f16"
    if cd == torch.float32 and pd == torch.float32:
        return "f32"
    return None


def unsupported_reason(model, batch_size):
    """None if Decoder(model, batch_size) applies, else why not."""
    from .mingru.minGRU import minGRU

    kind = _kind(model)
    f32 = kind == "f32"
    if kind is None:
        return ("Decoder needs bf16 activations (a minLM built with compute_dtype=torch.bfloat16, or one cast "
                "with .to(torch.bfloat16)), an fp32 model or a float16 one")
    if not 1 <= batch_size <= MAX_BATCH:
        return f"Decoder batch {batch_size} outside [1, {MAX_BATCH}]"
    D, Di, F, V = _widths(model)
    staged = MAX_STAGED if not f32 or batch_size <= 4 else MAX_STAGED // 2
    if D % 8 or D > MAX_DIM or Di % 8 or Di > staged or F % 8 or F > staged or V < 1:
        return (f"Decoder widths: dim {D} (multiple of 8, <= {MAX_DIM}), scan width {Di} and FeedForward width "
                f"{F} (multiples of 8, <= {staged})")
    for conv, _, gru, _, ff, dropout in model.layers:
        if conv is not None:
            return "Decoder does not run the causal conv (enable_conv)"
        if dropout is not None and model.training:
            return "Decoder runs dropout only in eval mode"
        if not isinstance(gru, minGRU) or gru.to_hidden_and_gate.weight.shape[0] != 2 * Di or \
                ff[0].weight.shape[0] != F:
            return "Decoder needs every layer at the same widths"
        if (Di != D) != isinstance(gru.to_out, torch.nn.Linear):
            return "Decoder needs to_out exactly when the scan width differs from dim"
    return None


def _f32(w):
    """w as an fp32 tensor: w itself if it is fp32, else a cached fp32 copy, re-made when w
    changes in place (the norm weights and embedding of a model cast to bf16)."""
    if w.dtype == torch.float32:
        return w
    cache = getattr(w, "_mg_f32", None)
    if cache is None or cache[0] != w._version or cache[1].device != w.device or cache[1].shape != w.shape:
        cache = (w._version, w.detach().float().contiguous())
        w._mg_f32 = cache
    return cache[1]


# Bumped whenever any module registers a parameter (a new Parameter object
# assigned, load_state_dict(assign=True)): decoders then re-gather the
# parameter objects they watch. In-place changes bump the tensors' own
# versions instead.
_PARAM_EPOCH = [0]


def _on_param_registered(module, name, param):
    _PARAM_EPOCH[0] += 1


torch.nn.modules.module.register_module_parameter_registration_hook(_on_param_registered)


class Decoder:
    def __init__(self, model, batch_size, graph=True, _weak=False):
        reason = unsupported_reason(model, batch_size)
        if reason:
            raise _lib.MingruHipError(reason)
        dev = model.token_emb.weight.device
        _lib.require_cuda(model.token_emb.weight)
        # the per-model cache of minLM.forward holds its decoders weakly referencing the model
        self._model = weakref.ref(model) if _weak else (lambda m=model: m)
        self.B, self.graph_enabled = batch_size, graph
        self.D, self.Di, self.F, self.V = _widths(model)
        self.kind = _kind(model)  # "bf16", "f32" (the *_f32 steps) or "f16" (the *_f16 steps)
        self.f32 = self.kind == "f32"
        et = {"bf16": torch.bfloat16, "f32": torch.float32, "f16": torch.float16}[self.kind]  # weights, outputs
        self.expanded = self.Di != self.D
        B, D, Di, F, V, L = self.B, self.D, self.Di, self.F, self.V, len(model.layers)
        self.device = dev
        self.tokens = torch.zeros(B, dtype=torch.int64, device=dev)
        self.x = [torch.zeros(B, D, device=dev) for _ in range(2)]
        self.pending = torch.zeros(B, D, dtype=et, device=dev)
        self.h = torch.zeros(B, Di, dtype=et, device=dev) if self.expanded else None
        self.act = torch.zeros(B, F, dtype=et, device=dev)
        self.logits = torch.zeros(B, V, dtype=et, device=dev)
        self.state_all = torch.zeros(L, B, Di, device=dev)  # one tensor: one copy in or out for all layers
        self.state = list(self.state_all.unbind(0))
        self._graph = None
        self._weights = None
        self._returned = None  # hiddens forward_one returned last (their values still equal the state)
        self._params, self._epoch = None, -1  # the parameters the weights come from
        self._sig, self._sig_refs, self._wcache = None, None, None

    @property
    def model(self):
        m = self._model()
        if m is None:
            raise _lib.MingruHipError("the Decoder's model no longer exists")
        return m

    # -- weights: the bf16 copies the training path also uses; fp32 norm weights and embedding
    def _current_weights(self):
        m = self.model
        if self.kind != "bf16":  # the parameters themselves (fp32 norm weights and embedding)
            ws = []
            for _, norm, gru, ff_norm, ff, _ in m.layers:
                ws += [_f32(norm.weight), gru.to_hidden_and_gate.weight.detach(),
                       gru.to_out.weight.detach() if self.expanded else None, _f32(ff_norm.weight),
                       ff[0].weight.detach(), ff[0].bias.detach(), ff[2].weight.detach(), ff[2].bias.detach()]
            return ws + [_f32(m.token_emb.weight), _f32(m.norm.weight), m.to_logits.weight.detach()]
        ws = []
        for _, norm, gru, ff_norm, ff, _ in m.layers:
            ws += [_f32(norm.weight), bf16_copy(gru.to_hidden_and_gate.weight, dense=True),
                   bf16_copy(gru.to_out.weight, dense=True) if self.expanded else None, _f32(ff_norm.weight),
                   bf16_copy(ff[0].weight, dense=True), bf16_copy(ff[0].bias, dense=True),
                   bf16_copy(ff[2].weight, dense=True), bf16_copy(ff[2].bias, dense=True)]
        ws += [_f32(m.token_emb.weight), _f32(m.norm.weight), bf16_copy(m.to_logits.weight, dense=True)]
        return ws

    def _param_list(self):
        m = self.model
        ps = []
        for _, norm, gru, ff_norm, ff, _ in m.layers:
            ps += [norm.weight, gru.to_hidden_and_gate.weight] + ([gru.to_out.weight] if self.expanded else [])
            ps += [ff_norm.weight, ff[0].weight, ff[0].bias, ff[2].weight, ff[2].bias]
        return ps + [m.token_emb.weight, m.norm.weight, m.to_logits.weight]

    def _signature(self):
        """What _current_weights depends on, cheaply: each parameter's version and storage
        and the identity of its cached copies (bf16 copy, hi/lo pair, fp32 copy), which the
        fused optimizer step drops or keeps current when it changes a parameter through a
        raw pointer. Returns (ids, refs); refs keep the cached copies alive, so their ids
        are not reused while they are compared."""
        if self._params is None or self._epoch != _PARAM_EPOCH[0]:
            self._params, self._epoch = self._param_list(), _PARAM_EPOCH[0]
        refs = [(p.__dict__.get("_mg_bf16"), p.__dict__.get("_mg_pair"), p.__dict__.get("_mg_f32"))
                for p in self._params]
        sig = [(p._version, p.data_ptr(), id(r[0]), id(r[1]), id(r[2])) for p, r in zip(self._params, refs)]
        return sig, refs

    def _weights_now(self):
        """_current_weights(), recomputed only when the signature changed (a per-token
        rebuild of 8 cached copies per layer costs more host time than the token's kernels)."""
        sig, _ = self._signature()
        if self._wcache is None or sig != self._sig:
            self._wcache = self._current_weights()
            self._sig, self._sig_refs = self._signature()  # after the copies were (re)made
        return self._wcache

    def _launch(self, weights):
        L = lib()
        B, D, Di, F, V = self.B, self.D, self.Di, self.F, self.V
        st = stream_of(self.x[0])
        emb, final_norm, w_logits = weights[-3:]
        cur = 0
        for i in range(len(self.state)):
            norm_w, whg, w_to, ff_norm_w, w1, b1, w2, b2 = weights[8 * i: 8 * i + 8]
            nxt = 1 - cur
            if i == 0:  # the residual stream starts at the token's embedding row
                src = (ptr(self.tokens), ptr(emb), V, None, None)
            else:
                src = (None, None, 0, ptr(self.x[cur]), ptr(self.pending))
            if self.kind != "bf16":
                sfx = "_" + self.kind
                mingru, to_out, ff = (getattr(L, "mg_decode_" + n + sfx) for n in ("mingru", "to_out", "ff"))
                if self.expanded:
                    check(mingru(B, D, Di, *src, None, ptr(self.h), ptr(norm_w), ptr(whg), ptr(self.state[i]),
                                 FP32_EPS, st), "mg_decode_mingru" + sfx)
                    check(to_out(B, D, Di, *src, ptr(self.h), ptr(w_to), ptr(self.x[nxt]), st), "mg_decode_to_out" + sfx)
                else:
                    check(mingru(B, D, Di, *src, ptr(self.x[nxt]), None, ptr(norm_w), ptr(whg), ptr(self.state[i]),
                                 FP32_EPS, st), "mg_decode_mingru" + sfx)
                check(ff(B, D, F, ptr(self.x[nxt]), ptr(ff_norm_w), ptr(w1), ptr(b1), ptr(self.act), ptr(w2), ptr(b2),
                         ptr(self.pending), FP32_EPS, st), "mg_decode_ff" + sfx)
            else:
                if self.expanded:
                    check(L.mg_decode_mingru_expanded(B, D, Di, *src, ptr(self.h), ptr(norm_w), ptr(whg),
                                                      ptr(self.state[i]), FP32_EPS, st), "mg_decode_mingru_expanded")
                    check(L.mg_decode_to_out(B, D, Di, *src, ptr(self.h), ptr(w_to), ptr(self.x[nxt]), st),
                          "mg_decode_to_out")
                else:
                    check(L.mg_decode_mingru(B, D, *src, ptr(self.x[nxt]), ptr(norm_w), ptr(whg),
                                             ptr(self.state[i]), FP32_EPS, st), "mg_decode_mingru")
                check(L.mg_decode_ff(B, D, F, ptr(self.x[nxt]), ptr(ff_norm_w), ptr(w1), ptr(b1), ptr(self.act),
                                     ptr(w2), ptr(b2), ptr(self.pending), FP32_EPS, st), "mg_decode_ff")
            cur = nxt
        head = L.mg_decode_head if self.kind == "bf16" else getattr(L, "mg_decode_head_" + self.kind)
        check(head(B, D, V, ptr(self.x[cur]), ptr(self.pending), ptr(final_norm), ptr(w_logits), ptr(self.logits),
                   FP32_EPS, st), "mg_decode_head")

    def _capture(self, weights):
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        saved = self.state_all.clone()
        with torch.cuda.stream(side):
            self._launch(weights)  # warm-up launch outside the capture
        torch.cuda.current_stream(self.device).wait_stream(side)
        self.state_all.copy_(saved)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._launch(weights)
        self.state_all.copy_(saved)  # capture does not run the kernels, but keep the state exact
        self._graph, self._weights = g, weights

    def _run(self):
        weights = self._weights_now()
        if not self.graph_enabled:
            self._launch(weights)
            return
        if self._graph is None or any(a is not b for a, b in zip(weights, self._weights)):
            self._capture(weights)  # first step, or the weights were changed in place
        self._graph.replay()

    # -- public API
    def set_hiddens(self, hiddens):
        """Load the per-layer states from prev_hiddens ([B, 1, Di] each, as minLM returns them;
        any float dtype); None zeroes them (a sequence that starts here)."""
        self._returned = None
        if hiddens is None:
            self.state_all.zero_()
            return
        hiddens = list(hiddens)
        if len(hiddens) != len(self.state):
            raise _lib.MingruHipError(f"prev_hiddens has {len(hiddens)} entries for {len(self.state)} layers")
        torch._foreach_copy_(self.state, [h.reshape(self.B, self.Di) for h in hiddens])

    def hiddens(self):
        """The current per-layer states as prev_hiddens views ([B, 1, Di] fp32)."""
        return list(self.state_all.view(len(self.state), self.B, 1, self.Di).unbind(0))

    @torch.no_grad()
    def prefill(self, ids):
        """Parallel forward over the prompt ids [B, T] (reference generate.py:188);
        returns the logits of its last position [B, V] and sets the states."""
        logits, hiddens = self.model(ids, return_prev_hiddens=True)
        self.set_hiddens(hiddens)
        return logits[:, -1, :]

    @torch.no_grad()
    def step(self, tokens):
        """One token per batch row (tokens [B] int64, on the device) -> logits [B, V] (bf16;
        fp32 for an fp32 model, fp16 for a float16 one). The returned tensor is the decoder's
        buffer, overwritten by the next step."""
        self.tokens.copy_(tokens.reshape(self.B))
        self._returned = None
        self._run()
        return self.logits

    @torch.no_grad()
    def forward_one(self, tokens, prev_hiddens):
        """minLM.forward's one-token call (reference generate.py:199-203, mingru/minLM.py:97-138
        on one position): tokens [B, 1] and prev_hiddens (or None) -> (logits [B, 1, V] (bf16, fp32 for an fp32 model),
        next_prev_hiddens [B, 1, Di] fp32 per layer). Both are new tensors, so hiddens the
        caller keeps are never overwritten; when prev_hiddens are the hiddens this call
        returned last (the generation loop), the states are already in place and nothing is
        copied in."""
        ret = self._returned
        if not (ret is not None and prev_hiddens is not None and len(prev_hiddens) == len(ret)
                and all(a is b for a, b in zip(prev_hiddens, ret))):
            self.set_hiddens(prev_hiddens)
        self.tokens.copy_(tokens.reshape(self.B))
        self._run()
        out = self.state_all.clone()
        hiddens = list(out.view(len(self.state), self.B, 1, self.Di).unbind(0))  # one call for all layers
        self._returned = hiddens
        return self.logits.clone().view(self.B, 1, self.V), hiddens


_CACHE = weakref.WeakKeyDictionary()  # model -> {(batch, key): Decoder or the reason it does not apply}


def forward_one(model, tokens, prev_hiddens):
    """minLM.forward's one-token call on the decode kernels: (logits, next_prev_hiddens), or
    None where the Decoder does not apply to this model and batch. The model's decoders are
    made on first use and cached per batch; they refer to the model weakly, so the cache
    does not keep it alive. The applicability check is cached per batch under what can
    change it after construction (train/eval mode, parameter dtype and device, the
    compute dtype)."""
    from .mingru import _defaults

    B = tokens.shape[0]
    w = model.token_emb.weight
    key = (B, model.training, w.dtype, w.device, model.compute_dtype, _defaults.COMPUTE_DTYPE)
    per_model = _CACHE.setdefault(model, {})
    dec = per_model.get(key)
    if dec is None:
        reason = unsupported_reason(model, B)
        dec = reason if reason else Decoder(model, B, _weak=True)
        per_model[key] = dec
    if isinstance(dec, str):
        return None
    return dec.forward_one(tokens, prev_hiddens)
