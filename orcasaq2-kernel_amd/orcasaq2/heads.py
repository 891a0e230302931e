"""The output head and the embedding table (the reference's orcasaq2/heads.py surface).

* `lm_head` is an ordinary EXL3 linear when the pack quantizes it (`head_bits`), so
  Exl3Config.get_quant_method hands ParallelLMHead the linear method (config.py).
* `embed_tokens` is int8 rows with a per-row scale.  The table stays int8 in device memory
  and only the gathered rows are scaled (orcasaq2/heads.py:22-67); the gather runs in the
  HIP library (exl3_embed_int8_gather).
"""
from __future__ import annotations

import torch

from . import _native
from ._vllm_compat import QuantizeMethodBase
from .config import Exl3ShardParam


class Exl3EmbeddingMethod(QuantizeMethodBase):
    """int8 rows with a per-row scale, dequantized on the gathered rows."""

    def create_weights(self, layer, input_size_per_partition, output_partition_sizes,
                       input_size, output_size, params_dtype, **extra_weight_attrs):
        """Placeholders for the int8 form (qweight + scales) and a dense form; which one the
        pack carries is known only from what the loader delivers (orcasaq2/heads.py:29-37).
        extra_weight_attrs (vLLM's vocab-sharding loader) is deliberately not applied."""
        for suffix in ("qweight", "scales", "weight"):
            layer.register_parameter(suffix, Exl3ShardParam(suffix=suffix))
        layer.exl3_params_dtype = params_dtype

    def process_weights_after_loading(self, layer):
        """orcasaq2/heads.py:39-59: dense table, or int8 table + (vocab, 1) scales in the
        params dtype; errors for neither table or a table without scales."""
        q = layer.qweight.shards.get(0)
        s = layer.scales.shards.get(0)
        w = layer.weight.shards.get(0)
        dev = next((t.device for t in (q, w) if t is not None and t.device.type == "cuda"), None)
        if dev is None:
            dev = torch.device("cuda", torch.cuda.current_device()) if torch.cuda.is_available() \
                else torch.device("cpu")
        for p in ("qweight", "scales", "weight"):
            if hasattr(layer, p):
                delattr(layer, p)
        if q is None:
            if w is None:
                raise RuntimeError("embed_tokens: neither an int8 table nor a dense one loaded")
            layer.exl3_embed_q = None
            layer.exl3_embed = torch.nn.Parameter(w.to(dev), requires_grad=False)
            return
        if s is None:
            raise RuntimeError("embed_tokens: qweight without scales")
        layer.exl3_embed = None
        layer.exl3_embed_q = torch.nn.Parameter(q.to(dev).contiguous(), requires_grad=False)
        layer.exl3_embed_s = torch.nn.Parameter(
            s.to(dev, layer.exl3_params_dtype).reshape(-1, 1).contiguous(), requires_grad=False)

    def embedding(self, layer, input_: torch.Tensor) -> torch.Tensor:
        """table[ids] (dense) or int8 gather * per-row scale (orcasaq2/heads.py:61-67)."""
        if layer.exl3_embed_q is None:
            return layer.exl3_embed[input_]
        return _native.embed_int8(layer.exl3_embed_q, layer.exl3_embed_s, input_)

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
        """Tied-head use of the table: dequantize it and run a dense linear
        (orcasaq2/heads.py:69-75)."""
        if layer.exl3_embed_q is None:
            w = layer.exl3_embed
        else:
            w = layer.exl3_embed_q.to(x.dtype) * layer.exl3_embed_s
        out = torch.nn.functional.linear(x, w.to(x.dtype))
        return out + bias if bias is not None else out
