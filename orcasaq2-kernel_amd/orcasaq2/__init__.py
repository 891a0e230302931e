"""Serve EXL3 (exllamav3 trellis-quantized) checkpoints in vLLM on AMD MI355X.

Drop-in for the reference plugin jschang/OrcaSAQ2-kernel (package `orcasaq2`, entry point
`vllm.general_plugins: orcasaq2 = orcasaq2:register`): the same quantization config
(`quant_method: "exl3"`), the same per-shard capture of fused layers, the same
`orcasaq2::shard_gemm` custom op, and the same wrapping of `embed_tokens` / `lm_head`.
Underneath, the trellis arithmetic runs in libexl3hip.so -- hand-written gfx950 HIP
kernels behind a C ABI (include/exl3hip.h) -- instead of the exllamav3 CUDA extension.

  * Each shard of a fused vLLM layer (q/k/v in qkv_proj, gate/up in gate_up_proj) is its
    own EXL3 tensor with its own shape and K, so shards are kept separately and `apply`
    runs them side by side into one output.
  * Shapes are unknown until the weights arrive, so create_weights registers placeholders
    whose loader captures each shard.
Tensor parallelism is not implemented; TP > 1 raises rather than serving wrong numbers.
"""
import torch

from . import _native
from . import ops  # noqa: F401  (registers orcasaq2::shard_gemm and orcasaq2::shards_gemv)

BLOCK = 128
_HAD = {}


def _had(device, dtype):
    """Sylvester H128 / sqrt(128), cached per (device, dtype) (orcasaq2/__init__.py:33-40)."""
    key = (str(device), dtype)
    if key not in _HAD:
        h = torch.ones((1, 1))
        while h.shape[0] < BLOCK:
            h = torch.cat([torch.cat([h, h], 1), torch.cat([h, -h], 1)], 0)
        _HAD[key] = (h / BLOCK ** 0.5).to(device=device, dtype=dtype)
    return _HAD[key]


def _t128(x):
    """Blockwise size-128 Hadamard along the last dim (orcasaq2/__init__.py:43-46)."""
    s = x.shape
    return (x.reshape(*s[:-1], s[-1] // BLOCK, BLOCK) @ _had(x.device, x.dtype)).reshape(s)


def reconstruct_weight(trellis, suh, svh, mcg, mul1):
    """Deployed dense weight (out, in) fp16 = (diag(suh) H W_q H diag(svh))^T, with W_q from
    the HIP reconstruct kernel and the Hadamard/sign algebra in fp32
    (orcasaq2/__init__.py:49-61).  mcg/mul1 are the optional marker tensors (None when
    absent)."""
    from .ops import exl3_K

    ic, oc = suh.numel(), svh.numel()
    k = exl3_K(trellis)
    w = _native.reconstruct(trellis.contiguous(), k, _native.codebook_id(mcg is not None, mul1 is not None))
    assert w.shape == (ic, oc)
    w = w.float()
    w = _t128(w.t()).t() * suh.float().unsqueeze(1)
    w = _t128(w) * svh.float().unsqueeze(0)
    return w.t().contiguous().half()


def register():
    """vLLM general-plugin entry point (orcasaq2/__init__.py:64-94): fail fast if the HIP
    library cannot be loaded, register quant_method "exl3" (idempotent), and wrap the
    embedding / lm_head constructors."""
    from ._vllm_compat import init_logger, register_quantization_config

    logger = init_logger("vllm.orcasaq2")
    try:
        _native.lib()
    except Exception as e:
        raise RuntimeError(
            "orcasaq2 needs its HIP library (libexl3hip.so, gfx950 kernels), and loading it "
            f"failed: {type(e).__name__}: {e}\n"
            "Build it from this source tree with\n"
            "  python orcasaq2-kernel_amd/build_lib.py\n"
            "on a ROCm 7 machine (hipcc --offload-arch=gfx950)."
        ) from e

    from .config import Exl3Config

    try:
        register_quantization_config("exl3")(Exl3Config)
    except ValueError:
        return  # already registered in this process
    _patch_embedding_layers(logger)
    logger.info("orcasaq2 armed: quant_method 'exl3' is now loadable")


def _patch_embedding_layers(logger):
    """Give VocabParallelEmbedding and ParallelLMHead the quant config that model files
    construct them without (orcasaq2/__init__.py:97-153).  Each constructor is wrapped; the
    wrapper binds the call against the real signature and fills `quant_config` only when it
    is empty and the current vLLM config is an Exl3Config.  Idempotent."""
    import inspect

    from . import _vllm_compat as vc
    from .config import Exl3Config

    if getattr(vc.VocabParallelEmbedding, "_orca_patched", False):
        return

    def _current_exl3_config():
        try:
            cfg = vc.get_current_vllm_config()
        except Exception:
            return None
        qc = getattr(cfg, "quant_config", None) or \
            getattr(getattr(cfg, "model_config", None), "quant_config", None)
        return qc if isinstance(qc, Exl3Config) else None

    for cls in (vc.VocabParallelEmbedding, vc.ParallelLMHead):
        def make(orig_init):
            sig = inspect.signature(orig_init)

            def __init__(self, *args, **kwargs):
                # ParallelLMHead passes quant_config to its (also wrapped) parent
                # positionally, so bind against the signature instead of adding a keyword.
                try:
                    bound = sig.bind_partial(self, *args, **kwargs)
                except TypeError:
                    return orig_init(self, *args, **kwargs)
                if bound.arguments.get("quant_config") is None:
                    qc = _current_exl3_config()
                    if qc is not None:
                        bound.arguments["quant_config"] = qc
                        return orig_init(*bound.args, **bound.kwargs)
                return orig_init(self, *args, **kwargs)
            return __init__

        cls.__init__ = make(cls.__init__)
    vc.VocabParallelEmbedding._orca_patched = True
    logger.info("orcasaq2: embed_tokens / lm_head will receive the EXL3 quant config")
