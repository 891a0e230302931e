"""EXL3 pack loading (orcasaq2/loader.py): a small synthetic pack written with safetensors --
fused and plain trellis modules, both codebook flags, dense modules, a bias, an int8
embedding and a K=6 lm_head -- loaded through the plugin's own load protocol.

CPU tests check the grouping, shapes, K, flags and error messages; GPU tests run every
loaded module and compare with the oracle (trellis modules: per-row relative L2 <= 1e-3 in
fp64; dense modules: the same bar against an fp32 matmul; the int8 gather: bit-exact).
"""
import json
import os

import numpy as np
import pytest
import torch

from orcasaq2 import loader
from orcasaq2 import synthetic as syn

H, I, V = 256, 512, 1024      # hidden, intermediate, vocabulary of the mini model
KV = 128
REL_TOL = 1e-3


def _mods():
    """{pack module prefix: tensors} of the mini model (seed-fixed)."""
    g = torch.Generator().manual_seed(11)
    mods = {}

    def quant(prefix, ic, oc, K, mcg=False, seed=0):
        lin = syn.linear(ic, oc, K, seed=seed)
        t = {"trellis": lin["trellis"], "suh": lin["suh"], "svh": lin["svh"]}
        if mcg:
            t["mcg"] = torch.zeros(1, dtype=torch.int8)
        mods[prefix] = t

    def dense(prefix, ic, oc, bias=False):
        t = {"weight": (torch.randn(oc, ic, generator=g) / ic ** 0.5).half()}
        if bias:
            t["bias"] = torch.randn(oc, generator=g).half()
        mods[prefix] = t

    a0, m0 = "model.layers.0.self_attn", "model.layers.0.mlp"
    quant(f"{a0}.q_proj", H, H, 4, seed=1)
    quant(f"{a0}.k_proj", H, KV, 5, seed=2)
    quant(f"{a0}.v_proj", H, KV, 5, seed=3)
    quant(f"{a0}.o_proj", H, H, 3, seed=4)
    quant(f"{m0}.gate_proj", H, I, 3, mcg=True, seed=5)
    quant(f"{m0}.up_proj", H, I, 3, mcg=True, seed=6)
    quant(f"{m0}.down_proj", I, H, 2, seed=7)
    a1, m1 = "model.layers.1.self_attn", "model.layers.1.mlp"
    dense(f"{a1}.q_proj", H, H)
    dense(f"{a1}.k_proj", H, KV)
    dense(f"{a1}.v_proj", H, KV)
    dense(f"{a1}.o_proj", H, H, bias=True)
    quant(f"{m1}.gate_proj", H, I, 4, seed=8)
    quant(f"{m1}.up_proj", H, I, 2, seed=9)
    quant(f"{m1}.down_proj", I, H, 5, seed=10)
    mods["model.embed_tokens"] = {
        "qweight": torch.randint(-128, 128, (V, H), generator=g, dtype=torch.int8),
        "scales": (torch.rand(V, 1, generator=g) * 0.02).half(),
    }
    quant("lm_head", H, V, 6, seed=12)
    return mods


def write_pack(path, mods=None, sharded=False, config_in="quantization_config.json"):
    from safetensors.torch import save_file

    mods = _mods() if mods is None else mods
    tensors = {f"{p}.{s}": t.contiguous() for p, ts in mods.items() for s, t in ts.items()}
    manifest = {p: {"stored_tensors": {f"{p}.{s}": {"shape": list(t.shape), "dtype": str(t.dtype)}
                                       for s, t in ts.items()}} for p, ts in mods.items()}
    qc = {"quant_method": "exl3", "bits": 3.5, "head_bits": 6, "codebook": "3inst",
          "tensor_storage": manifest}
    os.makedirs(path, exist_ok=True)
    if config_in == "quantization_config.json":
        with open(os.path.join(path, "quantization_config.json"), "w") as f:
            json.dump(qc, f)
    elif config_in == "config.json":
        with open(os.path.join(path, "config.json"), "w") as f:
            json.dump({"model_type": "qwen3", "quantization_config": qc}, f)
    if not sharded:
        save_file(tensors, os.path.join(path, "model.safetensors"))
    else:
        names = sorted(tensors)
        parts = [names[0::2], names[1::2]]
        wm = {}
        for i, part in enumerate(parts):
            fn = f"model-{i + 1:05d}-of-00002.safetensors"
            save_file({n: tensors[n] for n in part}, os.path.join(path, fn))
            wm.update({n: fn for n in part})
        with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
            json.dump({"metadata": {}, "weight_map": wm}, f)
    return mods


@pytest.fixture(scope="module")
def pack_dir(tmp_path_factory):
    d = str(tmp_path_factory.mktemp("pack"))
    write_pack(d)
    return d


# ---------------------------------------------------------------- CPU

def test_read_config_and_plan(pack_dir):
    cfg = loader.read_config(pack_dir)
    assert cfg.bits == 3.5 and cfg.head_bits == 6 and cfg.codebook == "3inst"
    assert "model.layers.0.self_attn.q_proj" in cfg.quantized_prefixes
    assert "model.layers.1.self_attn.q_proj" not in cfg.quantized_prefixes
    p = loader.plan(loader.Pack(pack_dir))
    assert p["model.layers.0.self_attn.qkv_proj"] == [
        ("q", "model.layers.0.self_attn.q_proj"), ("k", "model.layers.0.self_attn.k_proj"),
        ("v", "model.layers.0.self_attn.v_proj")]
    assert [s for s, _ in p["model.layers.1.mlp.gate_up_proj"]] == [0, 1]
    assert p["model.layers.0.self_attn.o_proj"] == [(None, "model.layers.0.self_attn.o_proj")]
    assert set(p) == {f"model.layers.{i}.{m}" for i in (0, 1) for m in
                      ("self_attn.qkv_proj", "self_attn.o_proj", "mlp.gate_up_proj", "mlp.down_proj")} | \
        {"model.embed_tokens", "lm_head"}


def _check_structure(mods):
    qkv = mods["model.layers.0.self_attn.qkv_proj"]
    assert [(s.K, s.ic, s.oc, s.mcg) for s in qkv.exl3_shards] == \
        [(4, H, H, False), (5, H, KV, False), (5, H, KV, False)]
    gu = mods["model.layers.0.mlp.gate_up_proj"]
    assert [(s.K, s.oc, s.mcg, s.mul1) for s in gu.exl3_shards] == [(3, I, True, False)] * 2
    assert mods["model.layers.1.mlp.gate_up_proj"].exl3_shards[1].K == 2
    d1 = mods["model.layers.1.self_attn.qkv_proj"]
    assert d1.exl3_shards is None and tuple(d1.exl3_dense.shape) == (H + 2 * KV, H)
    o1 = mods["model.layers.1.self_attn.o_proj"]
    assert o1.bias is not None and o1.bias.shape == (H,)
    emb = mods["model.embed_tokens"]
    assert emb.exl3_embed_q.dtype == torch.int8 and tuple(emb.exl3_embed_s.shape) == (V, 1)
    head = mods["lm_head"]
    assert head.exl3_shards[0].K == 6 and head.exl3_shards[0].oc == V
    for m in mods.values():
        for p in ("trellis", "suh", "svh", "qweight"):
            assert not hasattr(m, p), "placeholders are dropped after loading"


def test_load_structure_cpu(pack_dir):
    _check_structure(loader.load(pack_dir, device="cpu"))


def test_load_sharded_pack_and_config_json(tmp_path):
    write_pack(str(tmp_path), sharded=True, config_in="config.json")
    mods = loader.load(str(tmp_path), device="cpu")
    _check_structure(mods)
    a = loader.load(str(tmp_path), device="cpu", only=["model.layers.0.mlp.down_proj"])
    assert list(a) == ["model.layers.0.mlp.down_proj"]
    assert torch.equal(a["model.layers.0.mlp.down_proj"].exl3_shards[0].trellis.cpu(),
                       _mods()["model.layers.0.mlp.down_proj"]["trellis"])


def test_load_errors(tmp_path):
    mods = _mods()
    del mods["model.layers.0.self_attn.o_proj"]["svh"]
    write_pack(str(tmp_path / "a"), mods)
    with pytest.raises(RuntimeError, match="has a trellis but no .svh"):
        loader.load(str(tmp_path / "a"), device="cpu")

    mods = _mods()
    del mods["model.layers.0.self_attn.v_proj"]
    write_pack(str(tmp_path / "b"), mods)
    with pytest.raises(RuntimeError, match=r"pack holds shards \['q', 'k'\]"):
        loader.load(str(tmp_path / "b"), device="cpu")

    mods = _mods()
    mods["model.layers.0.self_attn.k_proj"] = {"weight": torch.zeros(KV, H, dtype=torch.half)}
    write_pack(str(tmp_path / "c"), mods)
    with pytest.raises(RuntimeError, match="a fused layer must be all one kind"):
        loader.load(str(tmp_path / "c"), device="cpu")

    write_pack(str(tmp_path / "d"), _mods(), config_in=None)
    with pytest.raises(RuntimeError, match="no quantization_config"):
        loader.read_config(str(tmp_path / "d"))
    with open(tmp_path / "d" / "quantization_config.json", "w") as f:
        json.dump({"quant_method": "gptq"}, f)
    with pytest.raises(RuntimeError, match="is not 'exl3'"):
        loader.read_config(str(tmp_path / "d"))


# ---------------------------------------------------------------- GPU

@pytest.mark.gpu
@pytest.mark.parametrize("rows", [1, 3, 20])
def test_loaded_modules_match_oracle(pack_dir, oracle, native, rows):
    """Every loaded module on the GPU against the oracle (the fused layers' outputs are the
    shards' outputs concatenated in q/k/v, 0/1 order)."""
    mods = loader.load(pack_dir, device="cuda")
    src = _mods()
    pl = loader.plan(loader.Pack(pack_dir))
    g = torch.Generator().manual_seed(rows)
    for key, m in mods.items():
        if m.kind == "embedding":
            continue
        ic = (m.exl3_shards[0].ic if m.exl3_shards is not None else m.exl3_dense.shape[1])
        x = syn.activations(rows, ic, g)
        y = m(x.cuda()).float().cpu().numpy()
        col = 0
        for _, p in pl[key]:
            t = src[p]
            if "trellis" in t:
                K = t["trellis"].shape[-1] // 16
                ref = oracle.shard_gemm_ref(x.numpy(), t["trellis"], t["suh"].numpy(), t["svh"].numpy(),
                                            K, 1 if "mcg" in t else 0)
            else:
                ref = x.double().numpy() @ t["weight"].double().numpy().T
                if "bias" in t:
                    ref = ref + t["bias"].double().numpy()
            oc = ref.shape[1]
            err = oracle.rel_err_rows(y[:, col:col + oc], ref).max()
            assert err <= REL_TOL, f"{key} shard {p}: rel err {err}"
            col += oc
        assert col == y.shape[1]


@pytest.mark.gpu
def test_loaded_embedding_bit_exact(pack_dir):
    mods = loader.load(pack_dir, device="cuda", only=["model.embed_tokens"])
    emb = mods["model.embed_tokens"]
    t = _mods()["model.embed_tokens"]
    ids = torch.tensor([0, 5, 1023, 5, 77])
    got = emb(ids.cuda()).cpu()
    want = t["qweight"][ids].to(torch.half) * t["scales"][ids]
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert np.isfinite(got.float().numpy()).all()
