"""The drop-in plugin surface on the CPU (the reference's orcasaq2/config.py, heads.py and
__init__.py behaviour), with the package's vLLM stand-ins.

The product registers orcasaq2::shard_gemm / shards_gemv for the GPU only.  To drive
Exl3LinearMethod.apply here, this module registers a CPU kernel for those ops *inside the
test process*, computed by the CPU oracle -- the oracle is the checker, the product never
routes through it.
"""
import numpy as np
import pytest
import torch

import orcasaq2
from orcasaq2 import _vllm_compat as vc
from orcasaq2 import synthetic as syn
from orcasaq2.config import SHARD_IDS, Exl3Config, Exl3LinearMethod, Exl3ShardParam, _expand
from orcasaq2.heads import Exl3EmbeddingMethod
from orcasaq2.ops import exl3_K


@pytest.fixture(scope="module")
def cpu_ops(oracle):
    """Oracle-backed CPU kernels for the custom ops (host-logic tests only); `calls` records
    which op each call reached."""
    calls = []

    def one(x, trellis, suh, svh, oc, k, mcg, mul1):
        y = oracle.shard_gemm_ref(x.numpy(), trellis.numpy(), suh.numpy(), svh.numpy(), int(k), 1 if mcg else 0)
        return torch.from_numpy(y).to(torch.half)

    def single(*a):
        calls.append("shard_gemm")
        return one(*a)

    def many(name):
        def run(x, trellis, suh, svh, oc, k, mcg, mul1):
            calls.append(name)
            return torch.cat([one(x, *a) for a in zip(trellis, suh, svh, oc, k, mcg, mul1)], dim=1)
        return run

    torch.library.register_kernel("orcasaq2::shard_gemm", "cpu", single)
    torch.library.register_kernel("orcasaq2::shards_gemv", "cpu", many("shards_gemv"))
    torch.library.register_kernel("orcasaq2::shards_gemm", "cpu", many("shards_gemm"))
    return calls


def test_exl3_K_matches_reference_semantics():
    for last, want in [(32, 2), (48, 3), (56, 3.5), (64, 4), (80, 5), (96, 6), (24, 1.5), (40, 2.5)]:
        k = exl3_K(torch.empty(2, 2, last))
        assert k == want and isinstance(k, int) == float(want).is_integer()


def test_shard_slots():
    p = Exl3ShardParam(suffix="trellis")
    assert p.numel() == 0 and p.suffix == "trellis"
    assert [p.slot(s) for s in ("q", "k", "v")] == [0, 1, 2]
    assert p.slot(None) == 0 and p.slot(1) == 1 and p.slot((2, 3)) == 2
    with pytest.raises(ValueError, match="unknown shard id"):
        p.slot("z")
    assert SHARD_IDS["gate_up_proj"] == [0, 1]


def test_config_parsing_and_manifest():
    cfg = Exl3Config.from_config({"bits": 3.5, "tensor_storage": {
        "model.layers.0.mlp.gate_proj": {"stored_tensors": {"model.layers.0.mlp.gate_proj.trellis": {}}},
        "model.layers.0.linear_attn.in_proj_a": {"stored_tensors": {"x.weight": {}}}}})
    assert cfg.get_name() == "exl3" and cfg.bits == 3.5 and cfg.codebook == "mul1" and cfg.head_bits == 16
    assert cfg.quantized_prefixes == {"model.layers.0.mlp.gate_proj"}
    assert Exl3Config.get_config_filenames() == ["quantization_config.json"]
    assert torch.half in cfg.get_supported_act_dtypes() and cfg.get_min_capability() == 80
    assert _expand("m.l.0.mlp.gate_up_proj", "gate_up_proj") == ["m.l.0.mlp.gate_proj", "m.l.0.mlp.up_proj"]
    lin = vc.LinearBase(16, 16, quant_config=None)
    assert isinstance(cfg.get_quant_method(lin, "model.layers.0.mlp.gate_up_proj"), Exl3LinearMethod)
    assert isinstance(cfg.get_quant_method(lin, "model.layers.0.linear_attn.in_proj_a"), vc.UnquantizedLinearMethod)
    assert cfg.get_quant_method(torch.nn.Linear(2, 2), "x") is None


def test_tensor_parallel_refused():
    cfg = Exl3Config.from_config({})
    m = Exl3LinearMethod(cfg, "x")
    with pytest.raises(NotImplementedError, match="tensor parallelism"):
        m.create_weights(torch.nn.Module(), 64, [128], 128, 128, torch.half)


def _load(layer, lins, ids):
    for sid in ids:
        for name in ("trellis", "suh", "svh"):
            p = getattr(layer, name)
            p.weight_loader(p, lins[sid][name], sid)


def test_fused_layer_apply_matches_oracle(cpu_ops, oracle):
    cfg = Exl3Config.from_config({"bits": 4})
    spec = [("q", 256, 4), ("k", 128, 5), ("v", 128, 5)]
    lins = {sid: syn.linear(128, oc, K, seed=i) for i, (sid, oc, K) in enumerate(spec)}
    layer = vc.LinearBase(128, 512, bias=True, params_dtype=torch.float32, quant_config=cfg,
                          prefix="model.layers.0.self_attn.qkv_proj", output_partition_sizes=[256, 128, 128])
    _load(layer, lins, ["k", "v", "q"])
    layer.quant_method.process_weights_after_loading(layer)
    assert not hasattr(layer, "trellis") and layer.exl3_dense is None
    assert [s.oc for s in layer.exl3_shards] == [256, 128, 128]
    assert [s.K for s in layer.exl3_shards] == [4, 5, 5]
    assert all(s.suh.dtype == torch.half for s in layer.exl3_shards)
    layer.bias.data = torch.randn(512)
    # grouped decode-GEMV to 16 rows, grouped GEMM to GEMM_MAX_ROWS (144), per shard above
    route = {1: ["shards_gemv"], 3: ["shards_gemv"], 20: ["shards_gemm"], 144: ["shards_gemm"],
             145: ["shard_gemm"] * 3}
    for rows, want in route.items():
        x = torch.randn(rows, 128)
        cpu_ops.clear()
        y = layer(x)
        assert cpu_ops == want, (rows, cpu_ops)
        assert y.dtype == torch.float32 and y.shape == (rows, 512)
        col = 0
        for sid, oc, K in spec:
            ref = oracle.shard_gemm_ref(x.half().numpy(), lins[sid]["trellis"], lins[sid]["suh"].numpy(),
                                        lins[sid]["svh"].numpy(), K) + layer.bias.numpy()[col:col + oc]
            got = y[:, col:col + oc].numpy()
            assert np.abs(got - ref).max() <= 2e-3 * np.abs(ref).max()
            col += oc


def test_load_errors():
    cfg = Exl3Config.from_config({})
    layer = vc.LinearBase(128, 256, quant_config=cfg, prefix="p", output_partition_sizes=[128, 128])
    lin = syn.linear(128, 128, 3, seed=0)
    _load(layer, {0: lin}, [0])
    with pytest.raises(RuntimeError, match="shards give 128 outputs, layer wants 256"):
        layer.quant_method.process_weights_after_loading(layer)

    layer = vc.LinearBase(128, 128, quant_config=cfg, prefix="p")
    layer.trellis.weight_loader(layer.trellis, lin["trellis"], 0)
    layer.weight.weight_loader(layer.weight, torch.zeros(128, 128), 1)
    with pytest.raises(RuntimeError, match="trellis and 1 dense shards"):
        layer.quant_method.process_weights_after_loading(layer)

    layer = vc.LinearBase(128, 128, quant_config=cfg, prefix="p")
    with pytest.raises(RuntimeError, match="no trellis and no dense weight"):
        layer.quant_method.process_weights_after_loading(layer)

    layer = vc.LinearBase(128, 128, quant_config=cfg, prefix="p")
    layer.trellis.weight_loader(layer.trellis, lin["trellis"], None)
    layer.suh.weight_loader(layer.suh, lin["suh"], None)
    with pytest.raises(RuntimeError, match="trellis shard 0 arrived without its suh/svh"):
        layer.quant_method.process_weights_after_loading(layer)


def test_newer_loader_hooks_file_by_slot():
    """vLLM's BasevLLMParameter hooks (load_qkv_weight & co.) file the tensor like
    weight_loader does, with the shard id under either keyword."""
    p = Exl3ShardParam(suffix="suh")
    a, b = torch.ones(4), torch.zeros(4)
    p.load_qkv_weight(a, shard_id="v")
    p.load_merged_column_weight(b, loaded_shard_id=1)
    p.load_row_parallel_weight(b)
    assert p.shards[2] is a and p.shards[1] is b and p.shards[0] is b


def test_dense_fallback_layer():
    cfg = Exl3Config.from_config({})
    layer = vc.LinearBase(16, 24, quant_config=cfg, prefix="p", output_partition_sizes=[16, 8])
    w0, w1 = torch.randn(16, 16), torch.randn(8, 16)
    layer.weight.weight_loader(layer.weight, w1, 1)
    layer.weight.weight_loader(layer.weight, w0, 0)
    layer.quant_method.process_weights_after_loading(layer)
    assert layer.exl3_shards is None
    x = torch.randn(3, 16)
    assert torch.allclose(layer(x), x @ torch.cat([w0, w1]).T)


def test_embedding_method_load_paths():
    cfg = Exl3Config.from_config({})
    emb = vc.VocabParallelEmbedding(100, 8, params_dtype=torch.bfloat16, quant_config=cfg)
    assert isinstance(emb.quant_method, Exl3EmbeddingMethod)
    w = torch.randn(100, 8)
    emb.weight.weight_loader(emb.weight, w)
    emb.quant_method.process_weights_after_loading(emb)
    ids = torch.tensor([3, 7])
    assert torch.equal(emb(ids), w[ids])
    # int8 table without scales
    emb = vc.VocabParallelEmbedding(100, 8, params_dtype=torch.bfloat16, quant_config=cfg)
    emb.qweight.weight_loader(emb.qweight, torch.zeros(100, 8, dtype=torch.int8))
    with pytest.raises(RuntimeError, match="qweight without scales"):
        emb.quant_method.process_weights_after_loading(emb)
    emb = vc.VocabParallelEmbedding(100, 8, params_dtype=torch.bfloat16, quant_config=cfg)
    with pytest.raises(RuntimeError, match="neither an int8 table nor a dense one"):
        emb.quant_method.process_weights_after_loading(emb)
    # tied-head apply dequantizes the int8 table
    emb = vc.VocabParallelEmbedding(100, 8, params_dtype=torch.float32, quant_config=cfg)
    q = torch.randint(-128, 128, (100, 8), dtype=torch.int8)
    s = torch.rand(100)
    emb.qweight.weight_loader(emb.qweight, q)
    emb.scales.weight_loader(emb.scales, s)
    emb.quant_method.process_weights_after_loading(emb)
    x = torch.randn(2, 8)
    want = x @ (q.float() * s[:, None]).T
    assert torch.allclose(emb.quant_method.apply(emb, x), want, atol=1e-5)


def test_lm_head_gets_linear_method():
    cfg = Exl3Config.from_config({"head_bits": 6})
    assert isinstance(cfg.get_quant_method(object.__new__(vc.ParallelLMHead), "lm_head"), Exl3LinearMethod)


def test_register_and_patch_embedding_constructors(native):
    orcasaq2.register()
    assert vc.quant_registry()["exl3"] is Exl3Config
    orcasaq2.register()  # idempotent
    assert getattr(vc.VocabParallelEmbedding, "_orca_patched", False)
    cfg = Exl3Config.from_config({})

    class Cfg:
        quant_config = cfg

    with vc.set_current_vllm_config(Cfg()):
        emb = vc.VocabParallelEmbedding(64, 8)            # model code passes no quant_config
        head = vc.ParallelLMHead(64, 8, prefix="lm_head")  # forwards it positionally
    assert isinstance(emb.quant_method, Exl3EmbeddingMethod)
    assert isinstance(head.quant_method, Exl3LinearMethod)
    plain = vc.VocabParallelEmbedding(64, 8)              # no current EXL3 config: untouched
    assert plain.quant_method is None


_PLUGIN_PROCESS = r"""
import importlib, json, sys, tomllib
sys.path.insert(0, "orcasaq2-kernel_amd")
role = sys.argv[1]
# the entry point vLLM resolves in every process it starts (pyproject.toml, vllm.general_plugins)
spec = tomllib.load(open("pyproject.toml", "rb"))["project"]["entry-points"]["vllm.general_plugins"]["orcasaq2"]
mod, fn = spec.split(":")
register = getattr(importlib.import_module(mod), fn)
register()
register()                                   # vLLM may load general plugins more than once
import orcasaq2
from orcasaq2 import _vllm_compat as vc
from orcasaq2.config import Exl3Config, Exl3LinearMethod
from orcasaq2.heads import Exl3EmbeddingMethod
out = {"role": role, "registered": vc.quant_registry()["exl3"] is Exl3Config,
       "patched": bool(vc.VocabParallelEmbedding.__dict__.get("_orca_patched"))
                  and bool(vc.ParallelLMHead.__dict__.get("_orca_patched"))}
cfg = Exl3Config.from_config({"head_bits": 6})
class Cfg:
    quant_config = cfg
with vc.set_current_vllm_config(Cfg()):
    lin = vc.LinearBase(256, 384, quant_config=cfg, prefix="model.layers.0.self_attn.qkv_proj",
                        output_partition_sizes=[128, 128, 128])
    emb = vc.VocabParallelEmbedding(64, 8)
    head = vc.ParallelLMHead(64, 8, prefix="lm_head")
out["linear"] = type(lin.quant_method).__name__
out["placeholders"] = sorted(n for n, _ in lin.named_parameters())
out["embedding"] = isinstance(emb.quant_method, Exl3EmbeddingMethod)
out["lm_head"] = isinstance(head.quant_method, Exl3LinearMethod)
print(json.dumps(out))
"""


def test_plugin_in_fresh_processes_like_vllms_server_engine_and_worker():
    """vLLM loads general plugins in each process it starts (API server, engine core, each
    worker), each a fresh interpreter (reference orcasaq2/__init__.py:64-94).  Three fresh
    processes run at once, each resolving the pyproject entry point, calling register() twice
    and building stand-in layers: every one must import cleanly, register "exl3" once, wrap
    the embedding and lm_head constructors, and give a fused linear its six placeholders."""
    import json
    import os
    import subprocess
    import sys
    if sys.version_info < (3, 11):
        pytest.importorskip("tomli")
        code = _PLUGIN_PROCESS.replace("import importlib, json, sys, tomllib", "import importlib, json, sys\nimport tomli as tomllib")
    else:
        code = _PLUGIN_PROCESS
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    procs = [subprocess.Popen([sys.executable, "-c", code, role], cwd=root, stdout=subprocess.PIPE,
                              stderr=subprocess.PIPE, text=True)
             for role in ("api_server", "engine_core", "worker_0")]
    outs = []
    for p in procs:
        so, se = p.communicate(timeout=300)
        assert p.returncode == 0, se
        outs.append(json.loads(so.strip().splitlines()[-1]))
    assert [o["role"] for o in outs] == ["api_server", "engine_core", "worker_0"]
    for o in outs:
        assert o["registered"] and o["patched"], o
        assert o["linear"] == "Exl3LinearMethod", o
        assert o["placeholders"] == ["mcg", "mul1", "suh", "svh", "trellis", "weight"], o
        assert o["embedding"] and o["lm_head"], o


def test_product_op_has_no_cpu_path_without_the_test_kernel():
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, 'orcasaq2-kernel_amd'); import torch, orcasaq2\n"
            "x = torch.zeros(1, 128, dtype=torch.half); t = torch.zeros(8, 8, 64, dtype=torch.int16)\n"
            "s = torch.ones(128, dtype=torch.half)\n"
            "try:\n torch.ops.orcasaq2.shard_gemm(x, t, s, s, 128, 4.0, False, False)\nexcept Exception as e:\n"
            " print(type(e).__name__); sys.exit(0)\nsys.exit(1)\n")
    import os
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", code], cwd=root, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "NotImplementedError" in r.stdout or "RuntimeError" in r.stdout


def test_fused_gemm_routing_follows_the_measured_crossovers():
    """The op's choice between the fused decode-GEMM and the reconstruct branch, on the
    shapes whose crossovers were measured (orcasaq2.ops._fused_gemm_faster)."""
    from orcasaq2 import ops
    f = ops._fused_gemm_faster
    for rows in (17, 64, 80, 128, 144):
        assert f(rows, 17408, 5120)                    # down_proj: fused at every row count
    assert f(64, 5120, 6144) and not f(80, 5120, 6144) and not f(144, 5120, 6144)   # q / o-like
    assert f(128, 5120, 17408) and not f(144, 5120, 17408)                           # gate / up
    assert f(144, 512, 256) and f(144, 2048, 1024)     # unmeasured narrow inputs keep the fused path
    # above GEMM_MAX_ROWS: wide inputs (down_proj) fused to 2560 rows (config 3's 2048
    # included); gate/up-like shapes fused in (1536, 3072]; q/o-like shapes and narrow inputs
    # reconstruct
    r = ops._fused_route
    if not ops.GEMM_MAX_ROWS_SET:
        assert r(145, 17408, 5120) and r(512, 17408, 5120) and r(2048, 17408, 5120) and r(2560, 17408, 5120)
        assert not r(2561, 17408, 5120) and not r(3072, 17408, 5120) and not r(4096, 17408, 5120)
        assert r(2048, 5120, 17408) and r(3072, 5120, 17408)
        assert not r(1536, 5120, 17408) and not r(3073, 5120, 17408) and not r(4096, 5120, 17408)
    assert not r(145, 5120, 17408) and not r(1024, 5120, 17408)
    assert not r(2048, 5120, 6144) and not r(145, 512, 256) and not r(2048, 2048, 8192)
