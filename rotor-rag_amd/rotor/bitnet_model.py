"""BitNet-b1.58-2B-shape language model on MI355X, with the reference's loading and
forward surface (src/rotor/bitnet_model.py):

    model = load_bitnet_model(model_dir, use_gpu=True)          # :349
    logits, cache = model.forward(ids, past_kv_cache=cache, use_cache=True)   # :190
    tokens = model.generate_greedy(prompt_ids, max_new_tokens)

Checkpoint: ``model_dir/config.json`` (HF keys vocab_size, hidden_size,
num_hidden_layers, num_attention_heads, num_key_value_heads, intermediate_size; optional
rope_theta, rms_norm_eps, max_position_embeddings) and ``model_dir/model.safetensors`` with
the tensor names the reference reads (src/rotor/bitnet_model.py:100-188): ternary weights
as rotor/BitNet bytes ``[out, in/4]`` uint8 with a per-tensor ``weight_scale`` that
multiplies (the reference's convention, :179-188), bf16/fp32 norms and a bf16 embedding
tied to the LM head (:235).

Layer semantics of this build (the benchmark configuration, BitNet b1.58 structure):
    a = RMSNorm(x);  q, k, v = W2A8(a);  RoPE(q, k);  o = causal GQA attention
    x = x + Wo(RMSNorm_sub(o))
    f = RMSNorm(x);  x = x + Wd(RMSNorm_sub(relu(Wg f)^2 * Wu f))
The reference differs (no RoPE, no mask, SiLU gate, sub-norm after o_proj; see its
src/rotor/transformer.py:206-341); logits are therefore not comparable with it, only
the per-linear arithmetic is.  Every ternary linear runs in the HIP library; attention,
RoPE, norms and the LM head are HIP kernels of the same library.  The model runs on the
GPU only: ``use_gpu=False`` raises.
"""
from __future__ import annotations

import ctypes
import json
from pathlib import Path
from typing import Dict, Optional

import numpy as np

from . import _hip

TERNARY = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


def rope_table(max_len: int, head_dim: int, theta: float) -> np.ndarray:
    """(cos, sin) of pos * theta^(-2i/head_dim), [max_len, head_dim/2, 2] fp32 (computed in f64)."""
    i = np.arange(head_dim // 2, dtype=np.float64)
    inv = theta ** (-(2.0 * i) / head_dim)
    ang = np.arange(max_len, dtype=np.float64)[:, None] * inv[None, :]
    return np.stack([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)


class KVCache:
    """The KV cache of one sequence, read as the reference's list of per-layer caches
    (src/rotor/bitnet_model.py:223-228 builds it from src/rotor/transformer.py:250-257):
    ``len(cache)`` is the number of layers and ``cache[i]`` is ``{'k': K, 'v': V}``, float32
    arrays ``[1, n_kv_heads, length, head_dim]`` copied from the device on access (keys
    after RoPE, as this model attends with them).  ``cache.length`` is the number of
    cached tokens.

    The cache memory belongs to the model and holds one sequence at a time: a forward that
    starts a new sequence (no past cache) or a generate_greedy call overwrites it, which
    makes every older handle stale; passing a stale handle, or reading one, raises
    ValueError.  A handle of the current sequence may be reused to continue (or rewind)
    from its length."""

    def __init__(self, model: "BitNetModel", length: int, epoch: int):
        self.model = model
        self.length = length
        self.epoch = epoch

    def __len__(self):
        return self.model.n_layers

    def __getitem__(self, i):
        if isinstance(i, slice):
            return [self[j] for j in range(*i.indices(len(self)))]
        n = len(self)
        i = int(i)
        if i < 0:
            i += n
        if not 0 <= i < n:
            raise IndexError(f"layer {i} of a {n}-layer cache")
        return self.model._dev.layer_cache(i, self.length, self.epoch)

    def __iter__(self):
        for i in range(len(self)):
            yield self[i]


class BitNetModel:
    def __init__(self, config: Dict, use_gpu: bool = False):
        if not use_gpu:
            raise NotImplementedError("this build runs BitNetModel on the GPU only: pass use_gpu=True")
        self.config = dict(config)
        self.vocab_size = config["vocab_size"]
        self.d_model = config["d_model"]
        self.n_layers = config["n_layers"]
        self.n_heads = config.get("n_heads", 20)
        self.n_kv_heads = config.get("n_kv_heads", 4)   # reference default, src/rotor/bitnet_model.py:60
        self.d_ff = config.get("d_ff", 6912)
        self.head_dim = self.d_model // self.n_heads
        self.rope_theta = float(config.get("rope_theta", 500000.0))
        self.eps = float(config.get("rms_norm_eps", 1e-6))
        self.max_seq_len = int(config.get("max_seq_len", 2048))
        self.max_tokens = int(config.get("max_batch_tokens", 512))
        self.use_gpu = True
        from .gpu_layers import get_gpu, last_error

        self.gpu = get_gpu()
        if self.gpu is None:
            raise RuntimeError(f"BitNetModel(use_gpu=True): HIP backend unavailable: {last_error()}")
        self._dev = None

    # ------------------------------------------------------------------ loading
    def load_weights_from_safetensors(self, model_path: str):
        """Read the reference's tensor names (src/rotor/bitnet_model.py:92-188)."""
        import torch
        from safetensors import safe_open

        state = {}
        with safe_open(model_path, framework="pt") as f:
            for k in f.keys():
                state[k] = f.get_tensor(k)
        self.load_state(state)

    def load_state(self, state: Dict):
        """state: name -> torch tensor / numpy array, with the reference's names."""
        import torch

        def t(name):
            v = state[name]
            return v if isinstance(v, torch.Tensor) else torch.from_numpy(np.asarray(v))

        def f32(name):
            return t(name).to(torch.float32).contiguous()

        L = []
        for i in range(self.n_layers):
            p = f"model.layers.{i}"
            lw = {"input_norm": f32(f"{p}.input_layernorm.weight"),
                  "post_norm": f32(f"{p}.post_attention_layernorm.weight")}
            for name in TERNARY:
                grp = "self_attn" if name in ("q_proj", "k_proj", "v_proj", "o_proj") else "mlp"
                w = t(f"{p}.{grp}.{name}.weight").to(torch.uint8)
                scale = float(t(f"{p}.{grp}.{name}.weight_scale").to(torch.float32).reshape(-1)[0])
                lw[name] = (w if w.is_cuda else w.cpu().numpy(), scale)
            sub_a, sub_f = f"{p}.self_attn.attn_sub_norm.weight", f"{p}.mlp.ffn_sub_norm.weight"
            lw["attn_sub_norm"] = f32(sub_a) if sub_a in state else None
            lw["ffn_sub_norm"] = f32(sub_f) if sub_f in state else None
            L.append(lw)
        emb = t("model.embed_tokens.weight")
        if emb.dtype != torch.bfloat16:
            emb = emb.to(torch.bfloat16)
        self._dev = _DeviceModel(self, L, emb.contiguous(), f32("model.norm.weight"))

    # ------------------------------------------------------------------ inference
    def forward(self, input_ids, return_logits: bool = True, past_kv_cache: Optional[KVCache] = None,
                use_cache: bool = False):
        """Same contract as src/rotor/bitnet_model.py:190-244: ids [seq] or [batch, seq] ->
        (logits [seq, vocab] (or [batch, seq, vocab]), cache or None).  The KV cache stays
        on the device (a KVCache handle, readable as the reference's per-layer list); pass
        it back to continue a sequence.  A batch of several sequences runs them one after
        the other and keeps no cache (use_cache and past_kv_cache need batch 1)."""
        ids = np.asarray(input_ids)
        squeeze = ids.ndim == 1
        if ids.ndim not in (1, 2):
            raise ValueError("input_ids must be [seq] or [batch, seq]")
        if ids.ndim == 2 and ids.shape[0] != 1:
            # several sequences: each runs as its own sequence through the device cache, so
            # they can share a forward only when no cache is kept between calls
            if past_kv_cache is not None or use_cache:
                raise ValueError("batch > 1 with a KV cache: the device cache holds one sequence; "
                                 "run the sequences one at a time")
            for row in ids:
                self._dev._check_ids(row, 0)
            outs = [self.forward(row, return_logits)[0] for row in ids]
            return np.stack(outs), None
        if ids.ndim == 2:
            ids = ids[0]
        if past_kv_cache is not None:
            if past_kv_cache.model is not self or past_kv_cache.epoch != self._dev.epoch:
                raise ValueError("stale KV cache: the model's device cache now holds a newer sequence")
            start = past_kv_cache.length
        else:
            start = 0
            self._dev._check_ids(ids, 0)  # a rejected input leaves the cache (and its handles) as they were
            self._dev.epoch += 1  # a new sequence overwrites the device cache
        out = self._dev.forward(ids.astype(np.int32), start, return_logits)
        cache = KVCache(self, start + len(ids), self._dev.epoch) if use_cache else None
        if not squeeze:
            out = out[None]
        return out, cache

    def generate_greedy(self, prompt_ids, max_new_tokens: int, graph: bool = True, timings: Optional[dict] = None):
        """Greedy decoding with the KV cache, the protocol of TextGenerator
        (src/rotor/generation.py:244-279: the whole prompt first, then one token per step,
        argmax sampling :42).  The decode step is captured once as a HIP graph and replayed.
        When `timings` is a dict it receives prefill_ms and decode_ms (HIP events; graph
        capture excluded)."""
        return self._dev.generate(np.asarray(prompt_ids, dtype=np.int32), int(max_new_tokens), graph, timings)


class _DeviceModel:
    """Device-resident weights, KV cache and buffers, and the launch sequence."""

    def __init__(self, model: BitNetModel, layers, emb, final_norm):
        import torch

        self.m = model
        self.epoch = 0  # sequence counter of the device KV cache (see KVCache)
        # when a dict (off by default; for checking a run layer by layer against a CPU
        # restatement): a multi-token forward appends a device copy of every layer's attention
        # output to trace["attn"] and stores {"h": last row's hidden state before the final
        # norm [D], "logits": the fused LM head's logits of that row [V]} as trace["prefill"];
        # every one-token step (forward, or generate's decode steps, graph-replayed or not)
        # appends {"attn": [layers, H * hd] attention outputs (the split partials combined as
        # the o_proj prologue combines them), "h": [D], "logits": [V]} to trace["steps"]
        self.trace = None
        self._tbuf = None  # the trace's device buffers (allocated before any graph capture)
        hip = self.hip = model.gpu
        dev = self.device = hip.device
        D, F, H, Hkv, hd = model.d_model, model.d_ff, model.n_heads, model.n_kv_heads, model.head_dim
        self.D, self.F, self.H, self.Hkv, self.hd = D, F, H, Hkv, hd
        self.Lmax = model.max_seq_len
        if H * hd != D or H % Hkv:
            raise ValueError("unsupported head layout")
        self.layers = []
        for lw in layers:
            d = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in lw.items()
                 if k in ("input_norm", "post_norm", "attn_sub_norm", "ffn_sub_norm")}
            for name in TERNARY:
                wb, scale = lw[name]
                K = D if name != "down_proj" else F
                if name == "o_proj":
                    K = H * hd
                if isinstance(wb, torch.Tensor) and wb.is_cuda:
                    d[name] = hip.upload_device(wb, K, scale)
                else:
                    d[name] = hip.upload(np.asarray(wb), K, scale)
            d["kc"] = torch.zeros((Hkv, hd, self.Lmax), dtype=torch.float32, device=dev)
            d["vc"] = torch.zeros((Hkv, self.Lmax, hd), dtype=torch.float32, device=dev)
            self.layers.append(d)
        self.emb = emb.to(dev)
        self.final_norm = final_norm.to(dev)
        self.rope = torch.from_numpy(rope_table(self.Lmax, hd, model.rope_theta)).to(dev)
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self.ids = torch.zeros(max(self.Lmax, 1), dtype=torch.int32, device=dev)
        self.token = torch.zeros(1, dtype=torch.int32, device=dev)
        self.best = torch.zeros(1, dtype=torch.int64, device=dev)
        self.logits = torch.empty(model.vocab_size, dtype=torch.float32, device=dev)
        self.out_tokens = torch.zeros(self.Lmax, dtype=torch.int32, device=dev)
        lib = _hip.load()
        self.attn_ws_bytes = int(lib.rt_attention_decode_workspace(H, hd, self.Lmax))
        self.attn_ws = torch.zeros(self.attn_ws_bytes, dtype=torch.uint8, device=dev)  # decode partials
        cap = model.max_tokens
        self.act_d = hip.activations(cap, D)
        self.act_f = hip.activations(cap, F)
        self.state = {}
        # decode attention: True (default) combines the split-L partials and applies the
        # sub-norm inside every o_proj workgroup's prologue; False runs a separate combine
        # kernel and gives o_proj a plain RMSNorm prologue (one more launch per layer,
        # ~0.04 ms/token slower at 30 layers)
        self.attn_in_prologue = True
        # decode FFN: True (default, when the shapes allow) computes relu(g)^2 * u and its
        # per-block sums of squares in the gate/up GEMV's epilogue, so the down GEMV's
        # prologue only normalises and quantises; False runs the gate/up plan and lets the
        # down prologue form relu(g)^2 * u and reduce it
        self.ffn_pair = D % 64 == 0 and F % 64 == 0 and F <= 8192
        # decode: True (default, where the plan's shape allows it: hd 128, 4 query heads per KV
        # head, the q/k/v GEMV at 16 waves per workgroup) runs RoPE + KV append + the attention
        # partials inside the q/k/v GEMV's launch (rt_plan_attach_attention), one launch per
        # layer fewer; False launches rt_rope_attention_decode after the GEMV
        self.attn_in_qkv = True
        # decode, with the attention in the q/k/v launch: True (default, Lmax <= 640) also
        # combines the split partials there (shared by the workgroups of each KV group), writing
        # the attention output and its sums of squares, so o_proj's prologue only normalises and
        # quantises (RMSNORM_SSQ); False lets every o_proj workgroup combine the partials
        self.attn_combine_in_qkv = True
        # generate: True (default) lets every argmax write the chosen token's embedding row into
        # the decode input, so the decode step launches no embedding; False embeds the token
        # from its id at the start of every step
        self.embed_in_argmax = True
        # decode: True (default) lets o_proj and down also write the per-32 sums of squares of
        # the residual stream they produce, so the gate/up plan and the next layer's q/k/v
        # plan normalise from them (RMSNORM_SSQ) instead of reducing the row again
        self.ssq_chain = True

    def _state(self, M):
        st = self.state.get(M)
        if st is not None:
            return st
        import torch

        dev, D, F, H, Hkv, hd = self.device, self.D, self.F, self.H, self.Hkv, self.hd
        e = lambda *s: torch.empty(s, dtype=torch.float32, device=dev)
        st = {"h": e(M, D), "q": e(M, H * hd), "k": e(M, Hkv * hd), "v": e(M, Hkv * hd), "o": e(M, H * hd),
              "g": e(M, F), "u": e(M, F), "a": e(F),
              "ssq": torch.empty(F // 32, dtype=torch.float64, device=dev),
              "hssq": torch.empty((D + 31) // 32, dtype=torch.float64, device=dev)}
        st["qkv"], st["gu"], st["o_plan"], st["d_plan"] = [], [], [], []
        st["attn_fused"] = []  # per layer: the q/k/v plan runs the attention partials
        st["attn_comb"] = []   # per layer: ... and combines them into o[0] (sums of squares in ossq)
        st["gu_pair"] = []     # per layer (M > 64): the gate/up GEMM writes relu(g)^2 * u into am
        st["ossq"] = torch.empty(H * hd // 32, dtype=torch.float64, device=dev)
        hip, eps = self.hip, self.m.eps
        chain = M == 1 and self.ssq_chain
        for li, L in enumerate(self.layers):
            st["attn_fused"].append(False)
            st["attn_comb"].append(False)
            if M == 1:  # decode: one launch per plan, the input row is quantised in the GEMV prologue
                h, o, g, u = st["h"][0], st["o"][0], st["g"][0], st["u"][0]
                qkv_w, qkv_ys = [L["q_proj"], L["k_proj"], L["v_proj"]], [st["q"][0], st["k"][0], st["v"][0]]
                if chain and li > 0:  # the previous layer's down wrote the sums of squares of h
                    st["qkv"].append(hip.plan_fused(qkv_w, _hip.SRC_RMSNORM_SSQ, h, L["input_norm"], st["hssq"],
                                                    eps=eps, ys=qkv_ys))
                else:
                    st["qkv"].append(hip.plan_fused(qkv_w, _hip.SRC_RMSNORM, h, L["input_norm"], eps=eps, ys=qkv_ys))
                if self.attn_in_qkv and L["attn_sub_norm"] is not None and self.attn_in_prologue:
                    st["attn_fused"][li] = self._attach_attention(st["qkv"][li], L)
                if st["attn_fused"][li] and self.attn_combine_in_qkv and self.Lmax <= 640:
                    st["attn_comb"][li] = self._attach_combine(st["qkv"][li], o, st["ossq"])
                if st["attn_comb"][li]:
                    st["o_plan"].append(hip.plan_fused([L["o_proj"]], _hip.SRC_RMSNORM_SSQ, o, L["attn_sub_norm"],
                                                       st["ossq"], eps=eps, ys=[h], residuals=[h]))
                elif L["attn_sub_norm"] is not None and self.attn_in_prologue:
                    st["o_plan"].append(hip.plan_fused([L["o_proj"]], _hip.SRC_ATTN_NORM, self.attn_ws,
                                                       L["attn_sub_norm"], eps=eps, ys=[h], residuals=[h],
                                                       attn_head_dim=self.hd, attn_max_len=self.Lmax))
                elif L["attn_sub_norm"] is not None:
                    st["o_plan"].append(hip.plan_fused([L["o_proj"]], _hip.SRC_RMSNORM, o, L["attn_sub_norm"],
                                                       eps=eps, ys=[h], residuals=[h]))
                else:
                    st["o_plan"].append(hip.plan_fused([L["o_proj"]], _hip.SRC_QUANT, o, ys=[h], residuals=[h]))
                if chain:
                    st["o_plan"][li].set_output_ssq(st["hssq"])
                # the gate/up source: h after o_proj, normalised from o_proj's sums of squares
                gu_src = ((_hip.SRC_RMSNORM_SSQ, h, L["post_norm"], st["hssq"]) if chain
                          else (_hip.SRC_RMSNORM, h, L["post_norm"]))
                if L["ffn_sub_norm"] is not None and self.ffn_pair:
                    if "gate_up" not in L:  # the interleaved copy the pair plan runs (decode only)
                        L["gate_up"] = hip.interleave_gate_up(L["gate_proj"], L["up_proj"])
                    w_gu, scales = L["gate_up"]
                    st["gu"].append(hip.plan_gate_up(w_gu, scales, *gu_src, eps=eps, a=st["a"], ssq=st["ssq"]))
                    st["d_plan"].append(hip.plan_fused([L["down_proj"]], _hip.SRC_RMSNORM_SSQ, st["a"],
                                                       L["ffn_sub_norm"], st["ssq"], eps=eps, ys=[h], residuals=[h]))
                    if chain and li + 1 < len(self.layers):
                        st["d_plan"][li].set_output_ssq(st["hssq"])
                    continue
                st["gu"].append(hip.plan_fused([L["gate_proj"], L["up_proj"]], *gu_src, eps=eps, ys=[g, u]))
                if L["ffn_sub_norm"] is not None:
                    st["d_plan"].append(hip.plan_fused([L["down_proj"]], _hip.SRC_RELU2MUL_NORM, g, u,
                                                       L["ffn_sub_norm"], eps=eps, ys=[h], residuals=[h]))
                else:
                    st["d_plan"].append(hip.plan_fused([L["down_proj"]], _hip.SRC_RELU2MUL, g, u, ys=[h],
                                                       residuals=[h]))
                if chain and li + 1 < len(self.layers):
                    st["d_plan"][li].set_output_ssq(st["hssq"])
            else:
                st["qkv"].append(hip.plan_act([L["q_proj"], L["k_proj"], L["v_proj"]], [self.act_d] * 3, M,
                                              [st["q"], st["k"], st["v"]]))
                if M > 64 and L["ffn_sub_norm"] is not None and self.ffn_pair:
                    # one GEMM over the interleaved gate/up matrix writes relu(g)^2 * u (am)
                    if "gate_up" not in L:
                        L["gate_up"] = hip.interleave_gate_up(L["gate_proj"], L["up_proj"])
                    if "am" not in st:
                        st["am"] = e(M, F)
                    w_gu, scales = L["gate_up"]
                    st["gu"].append(hip.plan_act_gate_up(w_gu, scales, self.act_d, M, st["am"]))
                    st["gu_pair"].append(True)
                else:
                    st["gu_pair"].append(False)
                    st["gu"].append(hip.plan_act([L["gate_proj"], L["up_proj"]], [self.act_d] * 2, M,
                                                 [st["g"], st["u"]]))
        self.state[M] = st
        return st

    def _attach_attention(self, plan, L):
        """Attach the decode attention to layer L's q/k/v plan; False where the library does
        not run it in that plan's launch (head size, query heads per KV head, workgroup size),
        which leaves the separate rt_rope_attention_decode launch."""
        try:
            plan.attach_attention(L["kc"], L["vc"], self.rope, self.H, self.Hkv, self.hd, self.Lmax, self.pos,
                                  self.attn_ws)
        except RuntimeError as e:
            if "rt_plan_attach_attention" not in str(e):
                raise
            return False
        return True

    def _attach_combine(self, plan, out, ssq):
        """Let layer L's q/k/v plan also combine the attention partials (into out, sums of
        squares into ssq); False where the library refuses (the device cannot hold the launch's
        workgroups at once), which leaves the combine to o_proj's prologue."""
        try:
            plan.attention_combine(out, ssq)
        except RuntimeError as e:
            if "rt_plan_attention_combine" not in str(e):
                raise
            return False
        return True

    def attention_timeouts(self):
        """Attention waits that gave up in the q/k/v launches since the last call (never
        expected; synchronises the device).  Raises if there were any: results are wrong."""
        st = self.state.get(1)
        n = 0
        if st is not None:
            n = sum(p.attention_timeouts() for p, on in zip(st["qkv"], st["attn_fused"]) if on)
        if n:
            raise RuntimeError(f"{n} attention waits in the q/k/v launches gave up: the decode results are invalid")

    def _trace_bufs(self):
        if self._tbuf is None:
            import torch

            e = lambda *s: torch.empty(s, dtype=torch.float32, device=self.device)
            self._tbuf = {"attn": e(len(self.layers), self.H * self.hd), "h": e(self.D)}
        return self._tbuf

    def _trace_record(self, key):
        """Copies of the trace buffers and the logits after a forward (see self.trace)."""
        tb = self._tbuf
        rec = {"h": tb["h"].clone(), "logits": self.logits.clone()}
        if key == "steps":
            rec["attn"] = tb["attn"].clone()
            self.trace.setdefault("steps", []).append(rec)
        else:
            self.trace[key] = rec

    def _enqueue(self, M, pos_base, out_cap, embed=True, next_h=None):
        """Forward of the M tokens in ids[0:M] at position *pos; LM head + argmax of the last.
        embed=False: h already holds the (one) token's embedding, written by the previous
        forward's argmax (next_h = that h: the chosen token's embedding row is written there)."""
        hip, lib, ctx = self.hip, _hip.load(), self.hip.ctx
        st = self._state(M)
        tb = self._trace_bufs() if self.trace is not None else None
        h, q, k, v, o, g, u = st["h"], st["q"], st["k"], st["v"], st["o"], st["g"], st["u"]
        hip._bind_stream()
        chk = _hip.check
        if embed:
            chk(lib.rt_embed(ctx, self.emb.data_ptr(), self.m.vocab_size, self.D, self.ids.data_ptr(), M,
                             h.data_ptr()), "rt_embed")
        eps = self.m.eps
        fused = M == 1
        for li, L in enumerate(self.layers):
            if fused:
                st["qkv"][li].run()
            else:
                hip.act_rmsnorm_quantize(h, L["input_norm"], self.act_d, eps)
                st["qkv"][li].gemv()
            if M == 1:
                combine_here = False
                if not st["attn_fused"][li]:
                    # RoPE + KV append + split attention in one launch (else they ran in the
                    # q/k/v launch); o_proj's prologue combines the partials, or this launch does
                    combine_here = L["attn_sub_norm"] is None or not self.attn_in_prologue
                    chk(lib.rt_rope_attention_decode(ctx, q.data_ptr(), k.data_ptr(), v.data_ptr(), L["kc"].data_ptr(),
                                                     L["vc"].data_ptr(), self.rope.data_ptr(), self.H, self.Hkv,
                                                     self.hd, self.Lmax, self.pos.data_ptr(), self.attn_ws.data_ptr(),
                                                     self.attn_ws_bytes, o.data_ptr() if combine_here else None),
                        "rt_rope_attention_decode")
                if tb is not None and (combine_here or st["attn_comb"][li]):  # o[0] holds the output
                    tb["attn"][li].copy_(o[0])
                elif tb is not None:  # the attention output the o_proj prologue forms from the partials
                    chk(lib.rt_attention_decode_combine(ctx, self.attn_ws.data_ptr(), self.attn_ws_bytes, self.H,
                                                        self.hd, self.Lmax, tb["attn"][li].data_ptr()),
                        "rt_attention_decode_combine")
            else:
                chk(lib.rt_rope_kv_append(ctx, q.data_ptr(), k.data_ptr(), v.data_ptr(), L["kc"].data_ptr(),
                                          L["vc"].data_ptr(), self.rope.data_ptr(), M, self.H, self.Hkv, self.hd,
                                          self.Lmax, self.pos.data_ptr()), "rt_rope_kv_append")
                chk(lib.rt_attention(ctx, q.data_ptr(), L["kc"].data_ptr(), L["vc"].data_ptr(), o.data_ptr(), M,
                                     self.H, self.Hkv, self.hd, self.Lmax, self.pos.data_ptr()), "rt_attention")
                if self.trace is not None:  # per-layer attention outputs of a multi-token forward
                    self.trace.setdefault("attn", []).append(o.clone())
            if fused:
                st["o_plan"][li].run()
                st["gu"][li].run()
                st["d_plan"][li].run()
                continue
            if L["attn_sub_norm"] is not None:
                hip.act_rmsnorm_quantize(o, L["attn_sub_norm"], self.act_d, eps)
            else:
                hip.act_quantize(o, self.act_d)
            hip.linear_act(L["o_proj"], self.act_d, out=h, residual=h)
            hip.act_rmsnorm_quantize(h, L["post_norm"], self.act_d, eps)
            st["gu"][li].gemv()
            if st["gu_pair"][li]:  # the gate/up launch wrote relu(g)^2 * u: the same values, sub-normed
                hip.act_rmsnorm_quantize(st["am"], L["ffn_sub_norm"], self.act_f, eps)
            elif L["ffn_sub_norm"] is not None:
                hip.act_relu2_mul_norm_quantize(g, u, L["ffn_sub_norm"], self.act_f, eps)
            else:
                hip.act_relu2_mul_quantize(g, u, self.act_f)
            hip.linear_act(L["down_proj"], self.act_f, out=h, residual=h)
        if tb is not None:
            tb["h"].copy_(h[M - 1])
        chk(lib.rt_lm_head_argmax(ctx, self.emb.data_ptr(), h[M - 1].data_ptr(), self.final_norm.data_ptr(), eps,
                                  self.m.vocab_size, self.D, self.logits.data_ptr(), self.best.data_ptr(),
                                  self.token.data_ptr(), self.pos.data_ptr(), M, self.ids.data_ptr(),
                                  self.out_tokens.data_ptr(), pos_base, out_cap,
                                  next_h.data_ptr() if next_h is not None else None), "rt_lm_head_argmax")
        return st

    def layer_cache(self, li, length, epoch):
        """Layer li's cached K and V of the current sequence's first `length` tokens, as
        float32 [1, Hkv, length, hd] host arrays."""
        if epoch != self.epoch:
            raise ValueError("stale KV cache: the model's device cache now holds a newer sequence")
        L = self.layers[li]
        k = L["kc"][:, :, :length].transpose(1, 2)  # the device keeps keys [Hkv, hd, Lmax]
        v = L["vc"][:, :length, :]
        return {"k": k.cpu().numpy()[None], "v": v.cpu().numpy()[None]}

    def _check_ids(self, ids, start):
        if len(ids) == 0:
            raise ValueError("empty input")
        if start + len(ids) > self.Lmax:
            raise ValueError(f"sequence of {start + len(ids)} tokens exceeds max_seq_len={self.Lmax}")
        if len(ids) > self.m.max_tokens:
            raise ValueError(f"{len(ids)} tokens in one forward exceed max_batch_tokens={self.m.max_tokens}")
        if ids.min() < 0 or ids.max() >= self.m.vocab_size:
            raise ValueError("token id out of range")

    def forward(self, ids, start, return_logits):
        import torch

        self._check_ids(ids, start)
        M = len(ids)
        self.ids[:M].copy_(torch.from_numpy(ids))
        self.pos.fill_(start)
        st = self._enqueue(M, pos_base=1 << 30, out_cap=0)
        if M == 1:
            self.attention_timeouts()
        if self.trace is not None:
            self._trace_record("steps" if M == 1 else "prefill")
        h = st["h"]
        if M == 1:
            out = self.logits[None] if return_logits else self._final_norm(h)
        else:
            hn = self._final_norm(h)
            out = self._lm_head_all(hn) if return_logits else hn
        return out.cpu().numpy()

    def _final_norm(self, h):
        import torch

        ss = (h.double() ** 2).sum(-1, keepdim=True)
        norm = torch.sqrt((ss / h.shape[-1]).float() + self.m.eps)
        return (h / norm) * self.final_norm

    def _lm_head_all(self, hn, chunk=16384):
        # every position's logits (reference semantics); the hot decode path uses the
        # fused LM-head kernel for the last position only
        import torch

        out = torch.empty((hn.shape[0], self.m.vocab_size), dtype=torch.float32, device=self.device)
        for v0 in range(0, self.m.vocab_size, chunk):
            out[:, v0:v0 + chunk] = hn @ self.emb[v0:v0 + chunk].float().T
        return out

    def generate(self, prompt, n, graph, timings=None):
        import torch

        self._check_ids(prompt, 0)
        self.epoch += 1  # the prompt overwrites the device cache
        P = len(prompt)
        if P + n > self.Lmax:
            raise ValueError("prompt + new tokens exceed max_seq_len")
        self._state(P)
        if self.trace is not None:
            self._trace_bufs()  # before the capture (not in the graph's memory pool)
        # every forward's argmax writes the chosen token's embedding into the decode input h,
        # so the decode steps launch no embedding (embed_in_argmax)
        h1 = self._state(1)["h"][0] if self.embed_in_argmax else None
        emb1 = not self.embed_in_argmax
        g = None
        if n > 1 and graph:  # capture the decode step first (capture does not execute it)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._enqueue(1, pos_base=P - 1, out_cap=n, embed=emb1, next_h=h1)
        self.ids[:P].copy_(torch.from_numpy(prompt))
        self.pos.fill_(0)
        self.best.zero_()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        rec = self._trace_record if self.trace is not None else (lambda key: None)
        ev[0].record()
        self._enqueue(P, pos_base=P - 1, out_cap=n, next_h=h1)  # prefill; out_tokens[0]
        rec("steps" if P == 1 else "prefill")
        ev[1].record()
        for _ in range(n - 1):
            if g is not None:
                g.replay()
            else:
                self._enqueue(1, pos_base=P - 1, out_cap=n, embed=emb1, next_h=h1)
            rec("steps")
        ev[2].record()
        torch.cuda.synchronize()
        self.attention_timeouts()
        if timings is not None:
            timings["prefill_ms"] = ev[0].elapsed_time(ev[1])
            timings["decode_ms"] = ev[1].elapsed_time(ev[2])
        return self.out_tokens[:n].cpu().numpy().copy()


def config_from_hf(cfg: Dict) -> Dict:
    """HF config.json -> the model config dict (src/rotor/bitnet_model.py:368-375)."""
    return {
        "vocab_size": cfg["vocab_size"],
        "d_model": cfg["hidden_size"],
        "n_layers": cfg["num_hidden_layers"],
        "n_heads": cfg["num_attention_heads"],
        "n_kv_heads": cfg.get("num_key_value_heads", cfg["num_attention_heads"]),
        "d_ff": cfg["intermediate_size"],
        "rope_theta": cfg.get("rope_theta", 500000.0),
        "rms_norm_eps": cfg.get("rms_norm_eps", 1e-6),
        "max_seq_len": cfg.get("max_position_embeddings", 2048),
    }


def load_bitnet_model(model_dir: str, use_gpu: bool = False) -> BitNetModel:
    """src/rotor/bitnet_model.py:349-394: config.json + model.safetensors -> BitNetModel."""
    model_dir = Path(model_dir)
    with open(model_dir / "config.json") as f:
        cfg = json.load(f)
    model = BitNetModel(config_from_hf(cfg), use_gpu=use_gpu)
    model.load_weights_from_safetensors(str(model_dir / "model.safetensors"))
    return model
