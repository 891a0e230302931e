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
import functools
import inspect

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


def _require_library() -> None:
    """Fail at plugin registration, not in the middle of a forward pass, when the HIP
    library cannot be loaded (the reference fails there on a missing exllamav3 wheel,
    orcasaq2/__init__.py:74-85)."""
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


def register():
    """vLLM general-plugin entry point (reference orcasaq2/__init__.py:64-94): check the HIP
    library, register quant_method "exl3", and let embed_tokens / lm_head see the EXL3
    config.  A second call in the same process changes nothing."""
    from ._vllm_compat import init_logger, register_quantization_config
    from .config import Exl3Config

    logger = init_logger("vllm.orcasaq2")
    _require_library()
    try:
        register_quantization_config("exl3")(Exl3Config)
    except ValueError:   # vLLM refuses a name twice: this process is armed already
        return
    wrapped = _patch_embedding_layers(logger)
    logger.info("orcasaq2 armed: quant_method 'exl3' is now loadable (%s wrapped)", ", ".join(wrapped) or "nothing")


def _current_exl3_config():
    """The current vLLM config's quant config when it is an Exl3Config, else None."""
    from . import _vllm_compat as vc
    from .config import Exl3Config

    try:
        cfg = vc.get_current_vllm_config()
    except Exception:
        return None
    for holder in (cfg, getattr(cfg, "model_config", None)):
        qc = getattr(holder, "quant_config", None)
        if qc is not None:
            return qc if isinstance(qc, Exl3Config) else None
    return None


def _wrap_constructor(cls) -> bool:
    """Wraps cls.__init__ (once per class) so that a call which leaves `quant_config` empty
    gets the current EXL3 config.  The argument is found by its position in the
    constructor's signature: vLLM's ParallelLMHead hands it to its (also wrapped) parent
    positionally, model code usually omits it.  Returns False when there is nothing to do."""
    if cls.__dict__.get("_orca_patched"):
        return False
    orig = cls.__init__
    names = list(inspect.signature(orig).parameters)
    if "quant_config" not in names:
        return False
    at = names.index("quant_config")          # position counting `self`

    @functools.wraps(orig)
    def __init__(self, *args, **kwargs):
        positional = len(args) >= at
        if (args[at - 1] if positional else kwargs.get("quant_config")) is None:
            qc = _current_exl3_config()
            if qc is not None:
                if positional:
                    args = args[:at - 1] + (qc,) + args[at:]
                else:
                    kwargs["quant_config"] = qc
        orig(self, *args, **kwargs)

    cls.__init__ = __init__
    cls._orca_patched = True
    return True


def _patch_embedding_layers(logger) -> list[str]:
    """Model files build embed_tokens and lm_head without a quant config, so vLLM would never
    ask this plugin about them; wrap both constructors to supply the current EXL3 config
    when it was left out (reference orcasaq2/__init__.py:97-153).  Layers of other quant
    methods are untouched."""
    from . import _vllm_compat as vc

    wrapped = [cls.__name__ for cls in (vc.VocabParallelEmbedding, vc.ParallelLMHead) if _wrap_constructor(cls)]
    if wrapped:
        logger.info("orcasaq2: %s receive the EXL3 quant config", " and ".join(wrapped))
    return wrapped
