"""Quantization config and linear method for EXL3 checkpoints.

Keeps the interface of the reference's orcasaq2/config.py -- the class and method names,
the `SHARD_IDS` table, the placeholder/weight-loader protocol and the user-facing errors --
and runs every shard through the gfx950 HIP ops of orcasaq2/ops.py.

Load protocol (what vLLM does with a quantized layer):
  1. `create_weights` registers one empty placeholder per tensor name an EXL3 layer may
     carry (shapes and K are unknown until the pack is read);
  2. the model loader calls each placeholder's `weight_loader(param, tensor, shard_id)`
     once per stored tensor -- a fused layer (qkv_proj, gate_up_proj) receives one tensor
     per constituent, each its own EXL3 tensor with its own shape and K;
  3. `process_weights_after_loading` turns what arrived into typed shard records (or a
     dense weight for a layer the pack left unquantized) on the worker's GPU;
  4. `apply` runs the shards and returns their outputs side by side.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Iterable

import torch

from ._vllm_compat import (
    BasevLLMParameter,
    LinearBase,
    LinearMethodBase,
    ParallelLMHead,
    QuantizationConfig,
    QuantizeMethodBase,
    UnquantizedLinearMethod,
    VocabParallelEmbedding,
    init_logger,
)
from . import ops as _ops
from .ops import GEMV_MAX_ROWS, exl3_K  # noqa: F401  (importing ops registers the custom ops)

logger = init_logger(__name__)

# Shard ids vLLM's loader passes for the constituents of its fused layers, listed in the
# order vLLM concatenates their outputs (reference orcasaq2/config.py:19-25).
SHARD_IDS = {
    "qkv_proj": ["q", "k", "v"],
    "gate_up_proj": [0, 1],
    "in_proj_qkvz": [0, 1],
}

# Named shard id -> slot ("q" -> 0, "k" -> 1, "v" -> 2).
_NAMED_SLOT = {name: i for ids in SHARD_IDS.values() for i, name in enumerate(ids) if isinstance(name, str)}

# The names a fused vLLM module's constituents carry in an EXL3 pack (its manifest keys).
_PACK_NAMES = {
    "qkv_proj": ("q_proj", "k_proj", "v_proj"),
    "gate_up_proj": ("gate_proj", "up_proj"),
    "in_proj_qkvz": ("in_proj_qkv", "in_proj_z"),
}

# Tensor names a linear layer may receive: the EXL3 set, or a plain weight when the pack
# left the layer unquantized (reference orcasaq2/config.py:183-184).
LINEAR_TENSORS = ("trellis", "suh", "svh", "mcg", "mul1", "weight")


def shard_slot(shard_id) -> int:
    """Slot of a loader shard id: None -> 0 (an unfused layer), an int -> itself, a tuple
    (a consecutive range of shards) -> its first element, a name of SHARD_IDS -> its
    position; anything else is an error (reference orcasaq2/config.py:53-63)."""
    match shard_id:
        case None:
            return 0
        case int():
            return shard_id
        case tuple():
            return shard_id[0]
        case str() if shard_id in _NAMED_SLOT:
            return _NAMED_SLOT[shard_id]
    raise ValueError(f"unknown shard id {shard_id!r}")


class Exl3ShardParam(BasevLLMParameter):
    """An empty placeholder Parameter standing for every tensor of one name that a layer
    receives; the tensors themselves are kept in `shards` (slot -> tensor) as they arrive.

    It carries its own `weight_loader` so that vLLM's generic
    `param.weight_loader(param, tensor, shard_id)` call files the tensor by slot instead of
    copying it into a parameter of a fixed shape (reference orcasaq2/config.py:28-71).
    """

    def __new__(cls, suffix: str):
        return super().__new__(cls, data=torch.empty(0))

    def __init__(self, suffix: str):
        super().__init__(data=torch.empty(0), weight_loader=_capture)
        self.suffix = suffix
        self.shards: dict[int, torch.Tensor] = {}

    def slot(self, shard_id) -> int:
        return shard_slot(shard_id)

    def _receive(self, loaded_weight: torch.Tensor, **kw) -> None:
        _capture(self, loaded_weight, kw.get("shard_id", kw.get("loaded_shard_id")))

    # vLLM's newer BasevLLMParameter loading hooks all reduce to filing the tensor
    load_column_parallel_weight = _receive
    load_row_parallel_weight = _receive
    load_merged_column_weight = _receive
    load_qkv_weight = _receive


def _capture(param: Exl3ShardParam, loaded_weight: torch.Tensor, shard_id=None, **kw) -> None:
    """weight_loader of every placeholder: keep the tensor as stored, under its slot."""
    param.shards[shard_slot(shard_id)] = loaded_weight


# ---------------------------------------------------------------- placeholder helpers
# (shared with the embedding method in heads.py)

def add_placeholders(layer: torch.nn.Module, names: Iterable[str]) -> None:
    for name in names:
        layer.register_parameter(name, Exl3ShardParam(suffix=name))


def take_loaded(layer: torch.nn.Module, names: Iterable[str]) -> dict[str, dict[int, torch.Tensor]]:
    """What each placeholder received (slot -> tensor); the placeholders leave the layer."""
    got = {}
    for name in names:
        param = layer._parameters.pop(name, None)
        got[name] = dict(param.shards) if param is not None else {}
    return got


def target_device(tensors: Iterable[torch.Tensor]) -> torch.device:
    """The GPU the loader already placed any of `tensors` on; otherwise this worker's
    current GPU (the CPU only where no GPU exists, for host-side tests)."""
    for t in tensors:
        if t.device.type == "cuda":
            return t.device
    if torch.cuda.is_available():
        return torch.device("cuda", torch.cuda.current_device())
    return torch.device("cpu")


def frozen(t: torch.Tensor) -> torch.nn.Parameter:
    return torch.nn.Parameter(t, requires_grad=False)


# ---------------------------------------------------------------- config

def _trellis_modules(manifest: dict | None) -> set[str]:
    """Module prefixes whose stored tensors include a `.trellis`, from a pack's
    `tensor_storage` manifest (reference orcasaq2/config.py:89-93)."""
    found = set()
    for module, entry in (manifest or {}).items():
        stored = (entry or {}).get("stored_tensors") or {}
        if any(name.endswith(".trellis") for name in stored):
            found.add(module)
    return found


def _expand(prefix: str, leaf: str) -> list[str]:
    """Pack names of a vLLM module: a fused module's constituents, or the module itself
    (reference orcasaq2/config.py:154-163)."""
    members = _PACK_NAMES.get(leaf)
    if members is None:
        return [prefix]
    parent = prefix[: len(prefix) - len(leaf)]
    return [parent + m for m in members]


class Exl3Config(QuantizationConfig):
    """`quant_method: "exl3"`: exllamav3 trellis quantization at any per-tensor bitrate
    (reference orcasaq2/config.py:79-151)."""

    # quantization_config.json keys and their defaults
    _DEFAULTS = {"bits": 0.0, "codebook": "mul1", "head_bits": 16}

    def __init__(self, bits: float, codebook: str, head_bits: float, full_config: dict):
        super().__init__()
        self.bits = bits
        self.codebook = codebook
        self.head_bits = head_bits
        self.full_config = full_config
        self.quantized_prefixes = _trellis_modules(full_config.get("tensor_storage"))

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
        d = cls._DEFAULTS
        return cls(bits=float(config.get("bits", d["bits"])), codebook=config.get("codebook", d["codebook"]),
                   head_bits=float(config.get("head_bits", d["head_bits"])), full_config=config)

    def get_quant_method(self, layer: torch.nn.Module, prefix: str) -> QuantizeMethodBase | None:
        """Linear layers -> Exl3LinearMethod, unless the pack's manifest shows that none of the
        module's constituents holds a trellis (then vLLM's unquantized method); the lm_head
        -> Exl3LinearMethod (an ordinary EXL3 tensor when the recipe quantizes it); the
        embedding -> Exl3EmbeddingMethod; any other layer -> None
        (reference orcasaq2/config.py:122-148)."""
        if isinstance(layer, LinearBase):
            if self.quantized_prefixes:
                names = _expand(prefix, prefix.rsplit(".", 1)[-1])
                if self.quantized_prefixes.isdisjoint(names):
                    return UnquantizedLinearMethod()
            return Exl3LinearMethod(self, prefix)
        if isinstance(layer, ParallelLMHead):   # a subclass of VocabParallelEmbedding: test it first
            return Exl3LinearMethod(self, prefix)
        if isinstance(layer, VocabParallelEmbedding):
            from .heads import Exl3EmbeddingMethod
            return Exl3EmbeddingMethod()
        return None

    def get_scaled_act_names(self):
        return []


# ---------------------------------------------------------------- linear method

@dataclass(frozen=True)
class Exl3Shard:
    """One EXL3 tensor of a layer, on the device, ready for the ops: trellis int16
    (ic/16, oc/16, 16K) contiguous, suh (ic) and svh (oc) fp16, the codebook flags."""
    trellis: torch.Tensor
    suh: torch.Tensor
    svh: torch.Tensor
    K: int | float
    ic: int
    oc: int
    mcg: bool
    mul1: bool


def _shard(prefix: str, slot: int, got: dict[str, dict[int, torch.Tensor]], dev: torch.device) -> Exl3Shard:
    trellis = got["trellis"][slot]
    if slot not in got["suh"] or slot not in got["svh"]:
        raise RuntimeError(f"{prefix}: trellis shard {slot} arrived without its suh/svh")
    suh = got["suh"][slot].to(dev, torch.half).contiguous()
    svh = got["svh"][slot].to(dev, torch.half).contiguous()
    return Exl3Shard(trellis=trellis.to(dev).contiguous(), suh=suh, svh=svh, K=exl3_K(trellis),
                     ic=suh.numel(), oc=svh.numel(), mcg=slot in got["mcg"], mul1=slot in got["mul1"])


class Exl3LinearMethod(LinearMethodBase):
    """EXL3 linear: shards filed by slot at load, run through the HIP ops at apply."""

    def __init__(self, quant_config: Exl3Config, prefix: str = ""):
        self.quant_config = quant_config
        self.prefix = prefix

    def create_weights(self, layer, input_size_per_partition, output_partition_sizes,
                       input_size, output_size, params_dtype, **extra_weight_attrs):
        """Placeholders for every tensor an EXL3 layer or an unquantized one may bring; which
        kind the layer is shows only in what the loader delivers (reference
        orcasaq2/config.py:171-185)."""
        if input_size_per_partition != input_size or sum(output_partition_sizes) != output_size:
            raise NotImplementedError(
                "orcasaq2 does not implement tensor parallelism yet; serve with -tp 1 "
                "rather than silently producing wrong numbers"
            )
        add_placeholders(layer, LINEAR_TENSORS)
        layer.exl3_out_total = sum(output_partition_sizes)

    def process_weights_after_loading(self, layer) -> None:
        """layer.exl3_shards: the EXL3 shards in slot order (= vLLM's concat order), or
        layer.exl3_dense: the stacked plain weights of a layer the pack left unquantized
        (reference orcasaq2/config.py:188-226)."""
        got = take_loaded(layer, LINEAR_TENSORS)
        trellis, dense = got["trellis"], got["weight"]
        dev = target_device([*trellis.values(), *dense.values()])
        if trellis and dense:
            raise RuntimeError(f"{self.prefix}: {len(trellis)} trellis and {len(dense)} dense shards; "
                               "a fused layer must be all one kind or all the other")
        if not trellis and not dense:
            raise RuntimeError(f"{self.prefix}: no trellis and no dense weight loaded")
        if dense:
            layer.exl3_shards = None
            stacked = torch.cat([dense[s] for s in sorted(dense)], dim=0)
            layer.exl3_dense = frozen(stacked.to(dev).contiguous())
            return
        shards = [_shard(self.prefix, s, got, dev) for s in sorted(trellis)]
        total = sum(s.oc for s in shards)
        if total != layer.exl3_out_total:
            raise RuntimeError(f"{self.prefix}: shards give {total} outputs, layer wants "
                               f"{layer.exl3_out_total}")
        layer.exl3_dense = None
        layer.exl3_shards = shards

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
        """fp16 activations through every shard, outputs side by side in slot order, cast
        back to x.dtype, plus bias (reference orcasaq2/config.py:228-245).  A fused layer at
        <= GEMM_MAX_ROWS rows, or above it when every shard routes to the fused kernel, is one
        grouped op (decode-GEMV up to 16 rows, stream-K GEMM above) that writes the
        concatenated output in place."""
        if layer.exl3_shards is None:
            out = torch.nn.functional.linear(x, layer.exl3_dense.to(x.dtype))
            return out + bias if bias is not None else out
        out = self.apply_fp16(layer, x).to(x.dtype)
        return out + bias if bias is not None else out

    def apply_fp16(self, layer, x: torch.Tensor) -> torch.Tensor:
        """The shards' fp16 outputs of apply, before the cast to x.dtype and the bias."""
        if layer.exl3_shards is None:
            raise RuntimeError(f"{self.prefix}: a dense fallback layer has no fp16 EXL3 output")
        rows = x.numel() // x.shape[-1]
        xf = x.reshape(rows, x.shape[-1]).half()
        if not xf.is_contiguous():
            xf = xf.contiguous()
        shards = layer.exl3_shards
        if len(shards) > 1 and 0 < rows and (rows <= _ops.GEMM_MAX_ROWS or all(
                _ops._fused_route(rows, xf.shape[-1], s.oc) for s in shards)):
            grouped = torch.ops.orcasaq2.shards_gemv if rows <= GEMV_MAX_ROWS else torch.ops.orcasaq2.shards_gemm
            out = grouped(
                xf, [s.trellis for s in shards], [s.suh for s in shards], [s.svh for s in shards],
                [s.oc for s in shards], [float(s.K) for s in shards], [s.mcg for s in shards],
                [s.mul1 for s in shards])
        else:
            outs = [torch.ops.orcasaq2.shard_gemm(xf, s.trellis, s.suh, s.svh, s.oc, float(s.K), s.mcg, s.mul1)
                    for s in shards]
            out = outs[0] if len(outs) == 1 else torch.cat(outs, dim=-1)
        return out.reshape(*x.shape[:-1], out.shape[-1])
