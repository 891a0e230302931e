"""Quantization config and linear method for EXL3 checkpoints (the reference's
orcasaq2/config.py surface: same classes, names, load protocol and errors), running the
shards through the gfx950 HIP ops in orcasaq2/ops.py."""
from __future__ import annotations

from typing import Any

import torch

from ._vllm_compat import (
    BasevLLMParameter,
    LinearBase,
    LinearMethodBase,
    QuantizationConfig,
    QuantizeMethodBase,
    init_logger,
)
from . import ops as _ops
from .ops import GEMV_MAX_ROWS, exl3_K  # noqa: F401  (importing ops registers the custom ops)

logger = init_logger(__name__)

# vLLM fuses these layers; each constituent is its own EXL3 tensor, so a fused layer holds
# a list of shards in vLLM's output concat order (orcasaq2/config.py:19-25).
SHARD_IDS = {
    "qkv_proj": ["q", "k", "v"],
    "gate_up_proj": [0, 1],
    "in_proj_qkvz": [0, 1],
}


class Exl3ShardParam(BasevLLMParameter):
    """Placeholder parameter for a list of per-shard EXL3 tensors (orcasaq2/config.py:28-71).

    EXL3 shard shapes and K are known only once the checkpoint is read, and differ between
    the shards of a fused layer, so the Parameter is an empty dummy and the loaded tensors
    are kept in `shards`, keyed by slot.  It carries its own `weight_loader`, which claims
    vLLM's generic `param.weight_loader(param, loaded_weight, shard_id)` path.
    """

    def __new__(cls, **kwargs):
        return super().__new__(cls, data=torch.empty(0))

    def __init__(self, suffix: str):
        super().__init__(data=torch.empty(0), weight_loader=_capture)
        self.shards: dict[int, torch.Tensor] = {}
        self.suffix = suffix

    def slot(self, shard_id) -> int:
        """None -> 0, int -> itself, tuple -> its first element, a SHARD_IDS name -> its
        index (q/k/v -> 0/1/2); anything else is a ValueError (orcasaq2/config.py:53-63)."""
        if shard_id is None:
            return 0
        if isinstance(shard_id, int):
            return shard_id
        if isinstance(shard_id, tuple):
            return shard_id[0]
        for ids in SHARD_IDS.values():
            if shard_id in ids:
                return ids.index(shard_id)
        raise ValueError(f"unknown shard id {shard_id!r}")

    # vLLM's newer parameter hooks (orcasaq2/config.py:65-71)
    def load_column_parallel_weight(self, loaded_weight, **kw):
        _capture(self, loaded_weight, kw.get("shard_id", kw.get("loaded_shard_id")))

    load_row_parallel_weight = load_column_parallel_weight
    load_merged_column_weight = load_column_parallel_weight
    load_qkv_weight = load_column_parallel_weight


def _capture(param, loaded_weight, shard_id=None, **kw):
    """Keep a loaded shard as-is; its shape is whatever the checkpoint holds."""
    param.shards[param.slot(shard_id)] = loaded_weight


class Exl3Config(QuantizationConfig):
    """`quant_method: "exl3"` -- exllamav3 trellis quantization at any per-tensor bitrate
    (orcasaq2/config.py:79-151)."""

    def __init__(self, bits: float, codebook: str, head_bits: float, full_config: dict):
        super().__init__()
        self.bits = bits
        self.codebook = codebook
        self.head_bits = head_bits
        self.full_config = full_config
        ts = full_config.get("tensor_storage") or {}
        self.quantized_prefixes = {
            k for k, v in ts.items()
            if any(n.endswith(".trellis") for n in (v.get("stored_tensors") or {}))
        }

    def __repr__(self):
        return (f"Exl3Config(bits={self.bits}, codebook={self.codebook!r}, "
                f"head_bits={self.head_bits}, quantized={len(self.quantized_prefixes)})")

    @classmethod
    def get_name(cls):
        return "exl3"

    @classmethod
    def get_supported_act_dtypes(cls):
        return [torch.half, torch.bfloat16]

    @classmethod
    def get_min_capability(cls):
        # vLLM compares this with its device-capability number; the reference's 80 is kept
        # so the same vLLM check passes wherever the reference's did.
        return 80

    @staticmethod
    def get_config_filenames():
        return ["quantization_config.json"]

    @classmethod
    def from_config(cls, config: dict[str, Any]):
        return cls(bits=float(config.get("bits", 0.0)),
                   codebook=config.get("codebook", "mul1"),
                   head_bits=float(config.get("head_bits", 16)),
                   full_config=config)

    def get_quant_method(self, layer: torch.nn.Module, prefix: str) -> QuantizeMethodBase | None:
        """Linear layers -> Exl3LinearMethod (or unquantized when the manifest says the layer
        has no trellis); ParallelLMHead -> Exl3LinearMethod; VocabParallelEmbedding ->
        Exl3EmbeddingMethod; anything else -> None (orcasaq2/config.py:122-148)."""
        if not isinstance(layer, LinearBase):
            from ._vllm_compat import ParallelLMHead, VocabParallelEmbedding
            if isinstance(layer, ParallelLMHead):
                return Exl3LinearMethod(self, prefix)
            if isinstance(layer, VocabParallelEmbedding):
                from .heads import Exl3EmbeddingMethod
                return Exl3EmbeddingMethod()
            return None
        leaf = prefix.rsplit(".", 1)[-1]
        if self.quantized_prefixes:
            if not any(c in self.quantized_prefixes for c in _expand(prefix, leaf)):
                from ._vllm_compat import UnquantizedLinearMethod
                return UnquantizedLinearMethod()
        return Exl3LinearMethod(self, prefix)

    def get_scaled_act_names(self):
        return []


def _expand(prefix: str, leaf: str) -> list[str]:
    """Fused vLLM name -> the HF names its shards were stored under."""
    mapping = {
        "qkv_proj": ["q_proj", "k_proj", "v_proj"],
        "gate_up_proj": ["gate_proj", "up_proj"],
        "in_proj_qkvz": ["in_proj_qkv", "in_proj_z"],
    }
    if leaf in mapping:
        return [prefix[: -len(leaf)] + m for m in mapping[leaf]]
    return [prefix]


class Exl3LinearMethod(LinearMethodBase):
    """EXL3 linear: per-shard trellis capture at load, HIP shard GEMMs at apply."""

    def __init__(self, quant_config: Exl3Config, prefix: str = ""):
        self.quant_config = quant_config
        self.prefix = prefix

    def create_weights(self, layer, input_size_per_partition, output_partition_sizes,
                       input_size, output_size, params_dtype, **extra_weight_attrs):
        """Placeholders for both a trellis and a dense form of every shard; which one a
        layer holds is only known from what the loader delivers (orcasaq2/config.py:171-185)."""
        if input_size != input_size_per_partition or sum(output_partition_sizes) != output_size:
            raise NotImplementedError(
                "orcasaq2 does not implement tensor parallelism yet; serve with -tp 1 "
                "rather than silently producing wrong numbers"
            )
        for suffix in ("trellis", "suh", "svh", "mcg", "mul1", "weight"):
            layer.register_parameter(suffix, Exl3ShardParam(suffix=suffix))
        layer.exl3_out_total = sum(output_partition_sizes)

    def process_weights_after_loading(self, layer) -> None:
        """Builds layer.exl3_shards in slot order -- trellis int16 contiguous, suh/svh fp16,
        codebook flags from the presence of .mcg/.mul1, K from the trellis width -- on the
        worker's GPU, or layer.exl3_dense for an unquantized layer (orcasaq2/config.py:188-226)."""
        tr, suh, svh = layer.trellis.shards, layer.suh.shards, layer.svh.shards
        mcg, mul1 = layer.mcg.shards, layer.mul1.shards
        dense = layer.weight.shards
        slots = sorted(tr) or sorted(dense)
        dev = next((t.device for t in list(tr.values()) + list(dense.values())
                    if t.device.type == "cuda"), None)
        if dev is None:
            dev = torch.device("cuda", torch.cuda.current_device()) if torch.cuda.is_available() \
                else torch.device("cpu")

        def finish():
            for p in ("trellis", "suh", "svh", "mcg", "mul1", "weight"):
                if hasattr(layer, p):
                    delattr(layer, p)

        if not tr:
            if not dense:
                raise RuntimeError(f"{self.prefix}: no trellis and no dense weight loaded")
            layer.exl3_shards = None
            w = torch.cat([dense[i] for i in slots], 0) if len(slots) > 1 else dense[slots[0]]
            layer.exl3_dense = torch.nn.Parameter(w.contiguous().to(dev), requires_grad=False)
            finish()
            return
        if dense:
            raise RuntimeError(f"{self.prefix}: {len(tr)} trellis and {len(dense)} dense shards; "
                               "a fused layer must be all one kind or all the other")
        layer.exl3_dense = None
        layer.exl3_shards = [
            dict(trellis=tr[i].contiguous().to(dev), suh=suh[i].to(dev, torch.half).contiguous(),
                 svh=svh[i].to(dev, torch.half).contiguous(),
                 mcg=mcg.get(i) is not None, mul1=mul1.get(i) is not None,
                 K=exl3_K(tr[i]), ic=suh[i].numel(), oc=svh[i].numel())
            for i in slots
        ]
        got = sum(s["oc"] for s in layer.exl3_shards)
        if got != layer.exl3_out_total:
            raise RuntimeError(f"{self.prefix}: shards give {got} outputs, layer wants "
                               f"{layer.exl3_out_total}")
        finish()

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
        """fp16 activations through every shard, outputs concatenated in slot order, cast
        back to x.dtype, plus bias (orcasaq2/config.py:228-245).  A multi-shard layer at
        <= GEMM_MAX_ROWS rows runs as one grouped op (decode-GEMV up to 16 rows, stream-K
        GEMM above) that writes the concat in place."""
        if layer.exl3_shards is None:
            out = torch.nn.functional.linear(x, layer.exl3_dense.to(x.dtype))
            return out + bias if bias is not None else out
        rows = x.numel() // x.shape[-1]
        xf = x.reshape(rows, x.shape[-1]).half()
        if not xf.is_contiguous():
            xf = xf.contiguous()
        shards = layer.exl3_shards
        if len(shards) > 1 and 0 < rows <= _ops.GEMM_MAX_ROWS:
            grouped = torch.ops.orcasaq2.shards_gemv if rows <= GEMV_MAX_ROWS else torch.ops.orcasaq2.shards_gemm
            out = grouped(
                xf, [s["trellis"] for s in shards], [s["suh"] for s in shards],
                [s["svh"] for s in shards], [s["oc"] for s in shards],
                [float(s["K"]) for s in shards], [s["mcg"] for s in shards],
                [s["mul1"] for s in shards])
        else:
            outs = [torch.ops.orcasaq2.shard_gemm(
                xf, s["trellis"], s["suh"], s["svh"], s["oc"], float(s["K"]), s["mcg"], s["mul1"])
                for s in shards]
            out = outs[0] if len(outs) == 1 else torch.cat(outs, dim=-1)
        out = out.to(x.dtype).reshape(*x.shape[:-1], out.shape[-1])
        return out + bias if bias is not None else out
