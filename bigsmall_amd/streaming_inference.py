"""Streaming inference: decode one transformer layer at a time on demand
(mirrors bigsmall/streaming_inference.py:77-347).

`BigSmallStreamingModel(bs_path, hf_config_path, device="cuda", prefetch=1)`
builds the HuggingFace module with empty weights, materialises the non-layer
weights once, and patches every layer's forward so that its weights are
decoded into HBM right before it runs and released right after.

Prefetch: the reference runs a host thread that decodes layers on the CPU
ahead of the forward pass, for exactly one pass over the layers
(streaming_inference.py:287-308; a second pass then waits on an empty queue).
Here, when layer i's forward starts, layer (i + 1) mod n_layers is submitted
to the loader's worker thread (its compressed bytes are read into pinned
memory, copied on a side stream and decoded by one batched launch on the
loader's decode stream), so it overlaps layer i's forward, which runs on the
caller's stream, on every pass.
"""
from __future__ import annotations

import gc
from pathlib import Path
from typing import Optional

from .streaming import StreamingLoader


def _get_dotted_module(model, dotted_name: str):
    obj = model
    for p in dotted_name.split("."):
        obj = obj[int(p)] if p.isdigit() else getattr(obj, p)
    return obj


def _set_param_data(module, dotted_name: str, tensor) -> None:
    """Swap a parameter (or buffer) for `tensor` by dotted name (streaming_inference.py:47-69)."""
    import torch
    parts = dotted_name.split(".")
    obj = _get_dotted_module(module, ".".join(parts[:-1])) if len(parts) > 1 else module
    leaf = parts[-1]
    if isinstance(getattr(obj, leaf), torch.nn.Parameter):
        setattr(obj, leaf, torch.nn.Parameter(tensor, requires_grad=False))
    else:
        setattr(obj, leaf, tensor)


def _layer_prefix(layer_idx: int, layer_template: str = "model.layers.{}") -> str:
    return layer_template.format(layer_idx) + "."


class BigSmallStreamingModel:
    """Inference wrapper that decodes one transformer layer at a time into HBM.

    bs_path: .bs file or directory with bigsmall.index.json + shards.
    hf_config_path: local directory (or file) with the model's config.json.
    device: ROCm device. dtype: floating dtype of the weights (default bf16).
    layer_template: "model.layers.{}" (Llama/Phi) or "h.{}" (GPT-2).
    prefetch: 1 = decode layer i+1 while layer i runs; 0 = decode on demand.
    """

    def __init__(self, bs_path: str | Path, hf_config_path: str | Path, device: str = "cuda", dtype=None,
                 layer_template: str = "model.layers.{}", prefetch: int = 1):
        import torch
        from accelerate import init_empty_weights
        from transformers import AutoConfig, AutoModelForCausalLM

        self.device = device
        self.dtype = dtype if dtype is not None else torch.bfloat16
        self.layer_template = layer_template
        self.config = AutoConfig.from_pretrained(str(hf_config_path))
        with init_empty_weights():
            self.model = AutoModelForCausalLM.from_config(self.config)
        self.model.eval()
        self.loader = StreamingLoader(bs_path, device=device, dtype=self.dtype, prefetch=prefetch)
        self.prefetch = max(0, int(prefetch))
        self._pending: dict[int, object] = {}

        for name, tensor in self.loader.load_non_layer_tensors().items():
            _set_param_data(self.model, name, tensor)
        self.n_layers = self.loader.layer_count()
        for i in range(self.n_layers):
            layer_module = _get_dotted_module(self.model, _layer_prefix(i, layer_template).rstrip("."))
            for tname, _ in list(layer_module.named_parameters(recurse=True)):
                _set_param_data(layer_module, tname, torch.empty(0, dtype=self.dtype, device=device))
            for tname, b in list(layer_module.named_buffers(recurse=True)):
                if b.device.type == "meta":
                    _set_param_data(layer_module, tname, torch.zeros_like(b, device=device))
        # buffers created outside the layers (rotary inv_freq, ...) live on the host: move them
        for bname, b in list(self.model.named_buffers()):
            if b.device.type not in ("meta", torch.device(device).type):
                _set_param_data(self.model, bname, b.to(device))
        # tied weights that stayed on the meta device (e.g. lm_head tied to the embedding)
        if getattr(self.config, "tie_word_embeddings", False) and hasattr(self.model, "tie_weights"):
            self.model.tie_weights()
        for i in range(self.n_layers):
            self._patch_layer(i)

    # ------------------------------------------------------------------------
    def _layer_tensors(self, layer_idx: int) -> dict:
        handle = self._pending.pop(layer_idx, None)
        if handle is None:
            handle = self.loader.submit_layer(layer_idx)
        if self.prefetch and self.n_layers > 1:
            nxt = (layer_idx + 1) % self.n_layers
            if nxt not in self._pending:
                self._pending[nxt] = self.loader.submit_layer(nxt)
        return self.loader.collect(handle)

    def _patch_layer(self, layer_idx: int) -> None:
        import torch
        prefix = _layer_prefix(layer_idx, self.layer_template)
        layer_module = _get_dotted_module(self.model, prefix.rstrip("."))
        original_forward = layer_module.forward
        outer = self

        def streaming_forward(*args, **kwargs):
            tensors = outer._layer_tensors(layer_idx)
            for full_name, t in tensors.items():
                if full_name.startswith(prefix):
                    _set_param_data(layer_module, full_name[len(prefix):], t)
            out = original_forward(*args, **kwargs)
            for full_name in tensors:
                if full_name.startswith(prefix):
                    _set_param_data(layer_module, full_name[len(prefix):],
                                    torch.empty(0, dtype=outer.dtype, device=outer.device))
            del tensors
            return out

        layer_module.forward = streaming_forward

    @classmethod
    def from_pretrained(cls, bs_path: str | Path, hf_config_path: Optional[str | Path] = None,
                        device: str = "cuda", dtype=None, layer_template: str = "model.layers.{}",
                        prefetch: int = 1) -> "BigSmallStreamingModel":
        """hf_config_path defaults to the directory holding the .bs file(s) if it has a config.json."""
        bs_path = Path(bs_path)
        if not bs_path.exists():
            raise FileNotFoundError(f"BigSmallStreamingModel.from_pretrained: path {bs_path!r} does not exist")
        if hf_config_path is None:
            cand = bs_path if bs_path.is_dir() else bs_path.parent
            if not (cand / "config.json").exists():
                raise FileNotFoundError(f"BigSmallStreamingModel.from_pretrained: no config.json next to {cand!r};"
                                        " pass hf_config_path")
            hf_config_path = cand
        return cls(bs_path, hf_config_path, device=device, dtype=dtype, layer_template=layer_template,
                   prefetch=prefetch)

    def forward(self, *args, **kwargs):
        import torch
        with torch.no_grad():
            return self.model(*args, **kwargs)

    def generate(self, input_ids, max_new_tokens: int = 20, **kwargs):
        import torch
        kwargs.setdefault("do_sample", False)
        kwargs.setdefault("max_new_tokens", max_new_tokens)
        with torch.no_grad():
            return self.model.generate(input_ids.to(self.device), **kwargs)

    def close(self) -> None:
        for h in self._pending.values():
            try:
                self.loader.collect(h)
            except Exception:
                pass
        self._pending.clear()
        self.loader.close()
        gc.collect()
