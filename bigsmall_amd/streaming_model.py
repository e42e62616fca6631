"""StreamingGPT2: GPT-2 run layer by layer from a BigSmall container
(the reference's proof of concept, bigsmall/streaming_model.py:29-176).

Non-layer weights (wte, wpe, ln_f) are decoded once and stay resident. The
transformer blocks come from `StreamingLoader.iter_layers`, which keeps
`loader.prefetch` layers in flight: while block i runs on the caller's
stream, block i+1 is read from the file, copied host to device and decoded on
the loader's own stream. A block's tensors are dropped once it has run, and
their memory goes back to torch's caching allocator (the loader records them
on the caller's stream, so none is reused while queued work still reads it);
the reference instead runs a garbage collection and empties the device cache
after every layer (streaming_model.py:156-159).

The block is GPT-2's own arithmetic written with torch primitives, as in the
reference (streaming_model.py:84-132): pre-LN, causal multi-head
self-attention with HF's Conv1D weight layout (`weight` stored (in, out)),
the "gelu_new" MLP, residual sums. Tensor names follow the GPT-2 safetensors
layout: `wte.weight`, `wpe.weight`, `ln_f.*`, `h.<i>.<sub>.*`.
"""
from __future__ import annotations

import math
from typing import Optional

import torch


def _gelu_new(x: torch.Tensor) -> torch.Tensor:
    """GPT-2's tanh approximation of GELU (streaming_model.py:22-26)."""
    return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x.pow(3))))


class StreamingGPT2:
    """Run GPT-2 layer by layer from a `StreamingLoader` (same constructor
    arguments as bigsmall/streaming_model.py:29-69).

    loader: an initialised StreamingLoader; its `prefetch` sets how many
        blocks decode ahead of the one running.
    config: a transformers.GPT2Config. Without one, GPT2Config()'s defaults
        are used, which are GPT-2 small's (the reference downloads the "gpt2"
        config from the hub instead; there is no network access here).
    device: where activations and weights live.
    dtype: optional floating dtype for weights and activations (default: as stored).
    """

    def __init__(self, loader, config=None, device: str = "cpu", dtype: Optional[torch.dtype] = None):
        from transformers import GPT2Config
        self.loader = loader
        self.device = device
        self.dtype = dtype
        self.config = config or GPT2Config()
        self.n_head = self.config.n_head
        self.n_embd = self.config.n_embd
        if self.n_embd % self.n_head:
            raise ValueError(f"n_embd {self.n_embd} is not a multiple of n_head {self.n_head}")
        self.head_dim = self.n_embd // self.n_head
        self.ln_eps = self.config.layer_norm_epsilon
        nl = loader.load_non_layer_tensors()
        missing = [k for k in ("wte.weight", "wpe.weight", "ln_f.weight", "ln_f.bias") if k not in nl]
        if missing:
            raise KeyError(f"StreamingGPT2: the container has no {missing} (GPT-2 safetensors names expected)")
        self.wte_weight = self._cast(nl["wte.weight"])
        self.wpe_weight = self._cast(nl["wpe.weight"])
        self.ln_f_weight = self._cast(nl["ln_f.weight"])
        self.ln_f_bias = self._cast(nl["ln_f.bias"])
        del nl

    def _cast(self, t: torch.Tensor) -> torch.Tensor:
        if self.dtype is not None and t.is_floating_point():
            t = t.to(self.dtype)
        return t.to(self.device)

    def _layer_norm(self, x, w, b):
        return torch.nn.functional.layer_norm(x, (x.shape[-1],), weight=w, bias=b, eps=self.ln_eps)

    def _block_forward(self, x: torch.Tensor, L: dict, layer_idx: int) -> torch.Tensor:
        """One GPT-2 block on hidden state x with the tensors of layer `layer_idx`."""
        p = f"h.{layer_idx}."
        h = self._layer_norm(x, L[p + "ln_1.weight"], L[p + "ln_1.bias"])
        qkv = h @ L[p + "attn.c_attn.weight"] + L[p + "attn.c_attn.bias"]      # Conv1D: x @ W + b
        B, T, _ = qkv.shape
        q, k, v = qkv.split(self.n_embd, dim=2)
        q = q.view(B, T, self.n_head, self.head_dim).transpose(1, 2)
        k = k.view(B, T, self.n_head, self.head_dim).transpose(1, 2)
        v = v.view(B, T, self.n_head, self.head_dim).transpose(1, 2)
        # batched products take contiguous right operands
        att = (q @ k.transpose(-1, -2).contiguous()) / math.sqrt(self.head_dim)
        mask = torch.tril(torch.ones(T, T, device=x.device, dtype=torch.bool))
        att = torch.softmax(att.masked_fill(~mask, float("-inf")), dim=-1)
        if self.dtype is not None:
            att = att.to(self.dtype)
        ctx = (att @ v.contiguous()).transpose(1, 2).contiguous().view(B, T, self.n_embd)
        x = x + (ctx @ L[p + "attn.c_proj.weight"] + L[p + "attn.c_proj.bias"])
        h = self._layer_norm(x, L[p + "ln_2.weight"], L[p + "ln_2.bias"])
        fc = _gelu_new(h @ L[p + "mlp.c_fc.weight"] + L[p + "mlp.c_fc.bias"])
        return x + (fc @ L[p + "mlp.c_proj.weight"] + L[p + "mlp.c_proj.bias"])

    @torch.no_grad()
    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        """Logits (B, T, vocab) for input_ids (B, T) (streaming_model.py:136-165)."""
        if input_ids.dim() == 1:
            input_ids = input_ids.unsqueeze(0)
        input_ids = input_ids.to(self.device)
        B, T = input_ids.shape
        positions = torch.arange(T, device=self.device).unsqueeze(0).expand(B, T)
        x = self.wte_weight[input_ids] + self.wpe_weight[positions]
        if self.dtype is not None:
            x = x.to(self.dtype)
        for i, L in self.loader.iter_layers(progress=False):
            L = {k: self._cast(v) for k, v in L.items()}
            x = self._block_forward(x, L, i)
            del L
        x = self._layer_norm(x, self.ln_f_weight, self.ln_f_bias)
        return torch.nn.functional.linear(x, self.wte_weight)       # tied LM head: x @ wte^T

    @torch.no_grad()
    def generate_greedy(self, input_ids: torch.Tensor, max_new_tokens: int) -> torch.Tensor:
        """Greedy decode of max_new_tokens continuation tokens (streaming_model.py:167-176)."""
        if input_ids.dim() == 1:
            input_ids = input_ids.unsqueeze(0)
        seq = input_ids.to(self.device)
        for _ in range(max_new_tokens):
            logits = self.forward(seq)
            seq = torch.cat([seq, torch.argmax(logits[:, -1, :], dim=-1, keepdim=True)], dim=1)
        return seq


__all__ = ["StreamingGPT2"]
