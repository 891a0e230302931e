"""The embedding table and the output head (the reference's orcasaq2/heads.py surface).

* `lm_head` needs nothing here: when a pack quantizes it (`head_bits`) it is an ordinary
  EXL3 tensor, and Exl3Config.get_quant_method gives ParallelLMHead the linear method.
  `lm_head_topk` adds the argmax / top-k epilogue (exl3_topk) behind it for greedy and
  top-k decoding, on the fp16 logits the GEMV writes.
* `embed_tokens` arrives either as int8 rows with one scale per row or as a plain table.
  The int8 table stays int8 in device memory: a lookup gathers the requested rows and
  scales only those, in the HIP library (exl3_embed_int8_gather); a tied head dequantizes
  the table for its matmul (reference orcasaq2/heads.py:22-75).
"""
from __future__ import annotations

import torch

from . import _native
from ._vllm_compat import QuantizeMethodBase
from .config import add_placeholders, frozen, take_loaded, target_device

# Tensor names an embedding may receive: the int8 form, or a plain table.
EMBED_TENSORS = ("qweight", "scales", "weight")


class Exl3EmbeddingMethod(QuantizeMethodBase):
    """int8 rows with a per-row scale, dequantized on the gathered rows; or a plain table."""

    def create_weights(self, layer, input_size_per_partition, output_partition_sizes,
                       input_size, output_size, params_dtype, **extra_weight_attrs):
        """Placeholders for both forms (reference orcasaq2/heads.py:29-37).  vLLM's
        vocab-sharding loader in extra_weight_attrs is not installed: the placeholders carry
        their own loader."""
        add_placeholders(layer, EMBED_TENSORS)
        layer.exl3_params_dtype = params_dtype

    def process_weights_after_loading(self, layer):
        """exl3_embed_q (int8, vocab x dim) + exl3_embed_s (vocab x 1, params dtype), or
        exl3_embed (the plain table) (reference orcasaq2/heads.py:39-59)."""
        got = {name: by_slot.get(0) for name, by_slot in take_loaded(layer, EMBED_TENSORS).items()}
        table, scales, plain = got["qweight"], got["scales"], got["weight"]
        dev = target_device([t for t in (table, plain) if t is not None])
        if table is not None:
            if scales is None:
                raise RuntimeError("embed_tokens: qweight without scales")
            layer.exl3_embed = None
            layer.exl3_embed_q = frozen(table.to(dev).contiguous())
            layer.exl3_embed_s = frozen(scales.to(dev, layer.exl3_params_dtype).reshape(-1, 1).contiguous())
        elif plain is not None:
            layer.exl3_embed_q = None
            layer.exl3_embed = frozen(plain.to(dev))
        else:
            raise RuntimeError("embed_tokens: neither an int8 table nor a dense one loaded")

    def embedding(self, layer, input_: torch.Tensor) -> torch.Tensor:
        """Rows of the table for the token ids (reference orcasaq2/heads.py:61-67)."""
        if layer.exl3_embed_q is not None:
            return _native.embed_int8(layer.exl3_embed_q, layer.exl3_embed_s, input_)
        return layer.exl3_embed[input_]

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
        """The table as a tied output head: x times the (dequantized) table transposed
        (reference orcasaq2/heads.py:69-75)."""
        if layer.exl3_embed_q is not None:
            table = layer.exl3_embed_q.to(x.dtype) * layer.exl3_embed_s
        else:
            table = layer.exl3_embed
        out = torch.nn.functional.linear(x, table.to(x.dtype))
        return out if bias is None else out + bias


def lm_head_topk(layer, x: torch.Tensor, k: int = 1) -> tuple[torch.Tensor, torch.Tensor]:
    """The output head and its top-k epilogue: the quantized lm_head's fp16 logits for
    hidden states x (..., hidden) (its EXL3 linear method, reference orcasaq2/config.py:
    128-132), then each row's k largest (values fp16 and columns int64, largest first,
    equal logits by smaller column; k = 1 is greedy decoding's argmax), both on the current
    stream.  A head with a bias adds it to the fp16 logits first."""
    method = getattr(layer, "quant_method", None)
    if not hasattr(method, "apply_fp16"):
        raise RuntimeError("lm_head_topk: the layer does not use the EXL3 linear method")
    logits = method.apply_fp16(layer, x)
    bias = getattr(layer, "bias", None)
    if bias is not None:
        logits = logits + bias.to(torch.float16)
    return _native.topk(logits, k)
