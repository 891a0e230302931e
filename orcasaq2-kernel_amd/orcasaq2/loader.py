"""Stand-alone loading of an EXL3 pack through the plugin's own load protocol.

Under vLLM the model loader drives the plugin: it builds each layer through
`Exl3Config.get_quant_method(...).create_weights(...)`, hands every checkpoint tensor to
`param.weight_loader(param, tensor, shard_id)` -- with the fused layers' shard ids (q/k/v,
0/1) from the model's stacked-parameter table -- and finally calls
`process_weights_after_loading` (reference orcasaq2/config.py:167-226,
orcasaq2/heads.py:22-59).  This module does the same from a pack directory without vLLM,
so a real checkpoint can run through the same boundary (and the same HIP ops) in tests,
benchmarks or a custom runtime.

A pack directory holds
  * the quantization config: `quantization_config.json` (the file name
    `Exl3Config.get_config_filenames` gives, orcasaq2/config.py:111-113) or the
    `quantization_config` entry of `config.json`, with `quant_method: "exl3"` and an
    optional `tensor_storage` manifest (orcasaq2/config.py:86-93);
  * safetensors files (`model.safetensors`, or shards listed by
    `model.safetensors.index.json`), one tensor per `<module>.<suffix>`: `trellis`, `suh`,
    `svh`, `mcg`, `mul1` (codebook flags: presence is what counts), `weight` (a dense
    module), `bias`; the embedding as `qweight` + `scales` (int8 rows, one scale per row)
    or a dense `weight` (orcasaq2/heads.py:29-59).

Modules are grouped the way vLLM fuses them (`q_proj`/`k_proj`/`v_proj` -> `qkv_proj`
shards q/k/v, `gate_proj`/`up_proj` -> `gate_up_proj` shards 0/1, `in_proj_qkv`/`in_proj_z`
-> `in_proj_qkvz` shards 0/1; orcasaq2/config.py:19-25, 154-163).  A module whose name ends
in `embed_tokens` gets the embedding method, everything else the linear method (which also
takes dense modules and lm_head, orcasaq2/config.py:128-132, 202-210).
"""
from __future__ import annotations

import json
import os
from collections import OrderedDict

import torch

from .config import Exl3Config, Exl3LinearMethod, SHARD_IDS

# HF module name -> (vLLM fused module, shard id)
FUSED = {
    "q_proj": ("qkv_proj", "q"), "k_proj": ("qkv_proj", "k"), "v_proj": ("qkv_proj", "v"),
    "gate_proj": ("gate_up_proj", 0), "up_proj": ("gate_up_proj", 1),
    "in_proj_qkv": ("in_proj_qkvz", 0), "in_proj_z": ("in_proj_qkvz", 1),
}
LINEAR_SUFFIXES = ("trellis", "suh", "svh", "mcg", "mul1", "weight")
EMBED_SUFFIXES = ("qweight", "scales", "weight")


def read_config(path: str) -> Exl3Config:
    """The pack's quantization config as an Exl3Config."""
    for fn in Exl3Config.get_config_filenames():
        p = os.path.join(path, fn)
        if os.path.exists(p):
            with open(p) as f:
                qc = json.load(f)
            break
    else:
        p = os.path.join(path, "config.json")
        qc = None
        if os.path.exists(p):
            with open(p) as f:
                qc = json.load(f).get("quantization_config")
        if qc is None:
            raise RuntimeError(f"{path}: no quantization_config.json and no quantization_config "
                               "in config.json")
    method = qc.get("quant_method", "exl3")
    if method != Exl3Config.get_name():
        raise RuntimeError(f"{path}: quant_method {method!r} is not {Exl3Config.get_name()!r}")
    return Exl3Config.from_config(qc)


class Pack:
    """Index of the tensors of a pack directory (names -> safetensors file); tensors are
    read one at a time, so a pack larger than host memory loads layer by layer."""

    def __init__(self, path: str):
        from safetensors import safe_open

        self.path = path
        index = os.path.join(path, "model.safetensors.index.json")
        if os.path.exists(index):
            with open(index) as f:
                wm = json.load(f)["weight_map"]
            files = sorted(set(wm.values()))
        else:
            files = sorted(f for f in os.listdir(path) if f.endswith(".safetensors"))
            wm = None
        if not files:
            raise RuntimeError(f"{path}: no .safetensors files")
        self.where: dict[str, str] = {}
        for fn in files:
            with safe_open(os.path.join(path, fn), framework="pt") as f:
                for k in f.keys():
                    if k in self.where:
                        raise RuntimeError(f"{path}: tensor {k} stored twice")
                    self.where[k] = fn
        if wm is not None:
            missing = [k for k, fn in wm.items() if self.where.get(k) != fn]
            if missing:
                raise RuntimeError(f"{path}: index lists {len(missing)} tensors its files do not "
                                   f"hold, e.g. {missing[0]}")

    def names(self) -> list[str]:
        return sorted(self.where)

    def get(self, name: str) -> torch.Tensor:
        from safetensors import safe_open

        with safe_open(os.path.join(self.path, self.where[name]), framework="pt") as f:
            return f.get_tensor(name)


def plan(pack: Pack) -> "OrderedDict[str, list[tuple[object, str]]]":
    """Module groups in load order: {vLLM module prefix: [(shard id, pack module prefix)]},
    shards in vLLM's concat order (q, k, v / 0, 1)."""
    mods: dict[str, set] = {}
    for name in pack.names():
        prefix, _, suffix = name.rpartition(".")
        if prefix and suffix in LINEAR_SUFFIXES + EMBED_SUFFIXES + ("bias",):
            mods.setdefault(prefix, set()).add(suffix)
    groups: dict[str, list] = {}
    for prefix in sorted(mods):
        head, _, leaf = prefix.rpartition(".")
        if leaf in FUSED:
            fused, sid = FUSED[leaf]
            key = f"{head}.{fused}" if head else fused
        else:
            key, sid = prefix, None
        groups.setdefault(key, []).append((sid, prefix))
    out: OrderedDict = OrderedDict()
    for key in sorted(groups):
        shards = groups[key]
        leaf = key.rpartition(".")[2]
        if leaf in SHARD_IDS:
            order = SHARD_IDS[leaf]
            shards.sort(key=lambda s: order.index(s[0]))
            got = [s[0] for s in shards]
            if got != order:
                raise RuntimeError(f"{key}: pack holds shards {got}, the fused layer needs {order}")
        out[key] = shards
    return out


class Exl3Module(torch.nn.Module):
    """One loaded module: the quant method plus the layer attributes it built.  forward()
    is the method's apply() for a linear module and its embedding() for the embedding."""

    def __init__(self, prefix: str, kind: str):
        super().__init__()
        self.prefix = prefix
        self.kind = kind            # "linear" or "embedding"
        self.quant_method = None
        self.bias = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.kind == "embedding":
            return self.quant_method.embedding(self, x)
        return self.quant_method.apply(self, x, self.bias)


def _shard_sizes(pack: Pack, prefix: str, kind: str) -> tuple[int, int]:
    """(in_features, out_features) of one stored module, from its tensors' shapes."""
    names = pack.where
    if kind == "embedding":
        t = pack.get(f"{prefix}.qweight") if f"{prefix}.qweight" in names else pack.get(f"{prefix}.weight")
        return t.shape[1], t.shape[0]
    if f"{prefix}.trellis" in names:
        for s in ("suh", "svh"):
            if f"{prefix}.{s}" not in names:
                raise RuntimeError(f"{prefix}: has a trellis but no .{s}")
        return pack.get(f"{prefix}.suh").numel(), pack.get(f"{prefix}.svh").numel()
    if f"{prefix}.weight" in names:
        w = pack.get(f"{prefix}.weight")
        return w.shape[1], w.shape[0]
    raise RuntimeError(f"{prefix}: neither .trellis nor .weight in the pack")


def load(path: str, device: torch.device | str | None = None, params_dtype: torch.dtype = torch.half,
         only: list[str] | None = None) -> "OrderedDict[str, Exl3Module]":
    """Loads the pack's modules (or those whose vLLM prefix is in `only`).  Tensors are read
    onto `device` (default: the current GPU); the quant methods then pin every module to the
    worker's GPU, as the reference's do (orcasaq2/config.py:191-197), and keep it on the CPU
    only where no GPU is visible.  Returns {vLLM module prefix: Exl3Module}."""
    cfg = read_config(path)
    pack = Pack(path)
    if device is None:
        device = torch.device("cuda", torch.cuda.current_device())
    device = torch.device(device)
    mods: OrderedDict = OrderedDict()
    for key, shards in plan(pack).items():
        if only is not None and key not in only:
            continue
        kind = "embedding" if key.rpartition(".")[2] == "embed_tokens" else "linear"
        m = Exl3Module(key, kind)
        sizes = [_shard_sizes(pack, p, kind) for _, p in shards]
        ics = {ic for ic, _ in sizes}
        if len(ics) != 1:
            raise RuntimeError(f"{key}: shards with different input widths {sorted(ics)}")
        ic, ocs = ics.pop(), [oc for _, oc in sizes]
        if kind == "embedding":
            from .heads import Exl3EmbeddingMethod
            m.quant_method = Exl3EmbeddingMethod()
            m.quant_method.create_weights(m, ic, ocs, ic, sum(ocs), params_dtype)
            suffixes = EMBED_SUFFIXES
        else:
            m.quant_method = Exl3LinearMethod(cfg, key)
            m.quant_method.create_weights(m, ic, ocs, ic, sum(ocs), params_dtype)
            suffixes = LINEAR_SUFFIXES
        biases = []
        for sid, p in shards:
            for s in suffixes:
                name = f"{p}.{s}"
                if name in pack.where:
                    param = getattr(m, s)
                    # as the vLLM loader does: the tensor goes to the worker's device first
                    param.weight_loader(param, pack.get(name).to(device), sid)
            if f"{p}.bias" in pack.where:
                biases.append(pack.get(f"{p}.bias"))
        m.quant_method.process_weights_after_loading(m)
        if biases:
            if len(biases) != len(shards):
                raise RuntimeError(f"{key}: bias on some shards only")
            m.bias = torch.nn.Parameter(torch.cat(biases).to(device, params_dtype), requires_grad=False)
        mods[key] = m
    return mods
