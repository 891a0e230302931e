"""vLLM names the plugin surface is written against, or minimal stand-ins without vLLM.

The reference imports these directly from vLLM (orcasaq2/config.py:5-12,
orcasaq2/heads.py:17, orcasaq2/__init__.py:65-66,114,122).  vLLM is an optional
dependency here: when it is importable the real classes are used and the plugin is a
drop-in; when it is not, the stand-ins below provide just enough of the same API (class
names, constructor and method signatures, the `weight_loader` protocol) for the plugin's
load -> process -> apply flow to be exercised, e.g. by the CPU tests.
"""
from __future__ import annotations

import logging
from typing import Any, Callable

import torch

try:  # pragma: no cover - exercised only where vLLM is installed
    from vllm.logger import init_logger
    from vllm.model_executor.layers.linear import LinearBase, LinearMethodBase
    from vllm.model_executor.layers.quantization.base_config import (
        QuantizationConfig,
        QuantizeMethodBase,
    )
    from vllm.model_executor.parameter import BasevLLMParameter
    from vllm.model_executor.layers.vocab_parallel_embedding import (
        ParallelLMHead,
        VocabParallelEmbedding,
    )
    from vllm.model_executor.layers.quantization import register_quantization_config
    from vllm.model_executor.layers.quantization.unquant import UnquantizedLinearMethod

    HAVE_VLLM = True
except Exception:  # vLLM absent: local stand-ins
    HAVE_VLLM = False

    def init_logger(name: str) -> logging.Logger:
        return logging.getLogger(name)

    class QuantizeMethodBase:
        """Stand-in for vllm...base_config.QuantizeMethodBase."""

        def create_weights(self, layer: torch.nn.Module, *args, **kwargs):
            raise NotImplementedError

        def apply(self, layer: torch.nn.Module, *args, **kwargs) -> torch.Tensor:
            raise NotImplementedError

        def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
            return

    class LinearMethodBase(QuantizeMethodBase):
        """Stand-in for vllm...linear.LinearMethodBase."""

    class QuantizationConfig:
        """Stand-in for vllm...base_config.QuantizationConfig."""

        def __init__(self):
            self.packed_modules_mapping: dict[str, list[str]] = {}

    class BasevLLMParameter(torch.nn.Parameter):
        """Stand-in for vllm.model_executor.parameter.BasevLLMParameter: a frozen
        Parameter that carries its own `weight_loader`."""

        def __new__(cls, data: torch.Tensor, **kwargs):
            return super().__new__(cls, data=data, requires_grad=False)

        def __init__(self, data: torch.Tensor, weight_loader: Callable):
            self._weight_loader = weight_loader

        @property
        def weight_loader(self):
            return self._weight_loader

    class LinearBase(torch.nn.Module):
        """Stand-in for vllm...linear.LinearBase: builds its weights through the quant
        method's create_weights and runs forward through quant_method.apply."""

        def __init__(self, input_size: int, output_size: int, bias: bool = False,
                     params_dtype: torch.dtype | None = None, quant_config=None,
                     prefix: str = "", output_partition_sizes: list[int] | None = None):
            super().__init__()
            self.input_size = input_size
            self.output_size = output_size
            self.input_size_per_partition = input_size
            self.output_partition_sizes = output_partition_sizes or [output_size]
            self.params_dtype = params_dtype or torch.get_default_dtype()
            self.prefix = prefix
            self.quant_method = (quant_config.get_quant_method(self, prefix)
                                 if quant_config is not None else UnquantizedLinearMethod())
            self.quant_method.create_weights(
                self, self.input_size_per_partition, self.output_partition_sizes,
                self.input_size, self.output_size, self.params_dtype)
            self.bias = (torch.nn.Parameter(torch.zeros(output_size, dtype=self.params_dtype),
                                            requires_grad=False) if bias else None)

        def forward(self, x: torch.Tensor) -> torch.Tensor:
            return self.quant_method.apply(self, x, self.bias)

    class UnquantizedLinearMethod(LinearMethodBase):
        """Stand-in for vllm...quantization.unquant.UnquantizedLinearMethod."""

        def create_weights(self, layer, input_size_per_partition, output_partition_sizes,
                           input_size, output_size, params_dtype, **extra_weight_attrs):
            w = torch.nn.Parameter(torch.empty(sum(output_partition_sizes),
                                               input_size_per_partition, dtype=params_dtype),
                                   requires_grad=False)
            layer.register_parameter("weight", w)

        def apply(self, layer, x, bias=None):
            return torch.nn.functional.linear(x, layer.weight, bias)

    class VocabParallelEmbedding(torch.nn.Module):
        """Stand-in for vllm...vocab_parallel_embedding.VocabParallelEmbedding."""

        def __init__(self, num_embeddings: int, embedding_dim: int,
                     params_dtype: torch.dtype | None = None, org_num_embeddings=None,
                     padding_size: int = 64, quant_config=None, prefix: str = ""):
            super().__init__()
            self.num_embeddings = num_embeddings
            self.embedding_dim = embedding_dim
            self.quant_config = quant_config
            self.prefix = prefix
            params_dtype = params_dtype or torch.get_default_dtype()
            self.quant_method = (quant_config.get_quant_method(self, prefix)
                                 if quant_config is not None else None)
            if self.quant_method is None:
                self.weight = torch.nn.Parameter(
                    torch.empty(num_embeddings, embedding_dim, dtype=params_dtype),
                    requires_grad=False)
            else:
                self.quant_method.create_weights(self, embedding_dim, [num_embeddings],
                                                 embedding_dim, num_embeddings, params_dtype)

        def forward(self, input_: torch.Tensor) -> torch.Tensor:
            if self.quant_method is None:
                return torch.nn.functional.embedding(input_, self.weight)
            return self.quant_method.embedding(self, input_)

    class ParallelLMHead(VocabParallelEmbedding):
        """Stand-in for vllm...vocab_parallel_embedding.ParallelLMHead.  It forwards
        quant_config to its parent positionally, as vLLM's does."""

        def __init__(self, num_embeddings: int, embedding_dim: int, bias: bool = False,
                     params_dtype: torch.dtype | None = None, org_num_embeddings=None,
                     padding_size: int = 64, quant_config=None, prefix: str = ""):
            super().__init__(num_embeddings, embedding_dim, params_dtype, org_num_embeddings,
                             padding_size, quant_config, prefix)

        def forward(self, input_):
            raise RuntimeError("LMHead's weights should be used in the sampler.")

    _QUANT_REGISTRY: dict[str, type] = {}

    def register_quantization_config(quantization: str):
        def _wrapper(cls):
            if quantization in _QUANT_REGISTRY:
                raise ValueError(f"The quantization method `{quantization}` is already exists.")
            _QUANT_REGISTRY[quantization] = cls
            return cls
        return _wrapper

_CURRENT_CONFIG: list[Any] = []


def get_current_vllm_config():
    """vllm.config.get_current_vllm_config when vLLM is present; otherwise the config set
    with `set_current_vllm_config` (a stand-in context manager for tests)."""
    if HAVE_VLLM:  # pragma: no cover
        from vllm.config import get_current_vllm_config as g
        return g()
    if not _CURRENT_CONFIG:
        raise RuntimeError("no current vLLM config")
    return _CURRENT_CONFIG[-1]


class set_current_vllm_config:
    """Context manager standing in for vllm.config.set_current_vllm_config."""

    def __init__(self, cfg):
        self.cfg = cfg

    def __enter__(self):
        _CURRENT_CONFIG.append(self.cfg)
        return self.cfg

    def __exit__(self, *exc):
        _CURRENT_CONFIG.pop()
        return False


def quant_registry() -> dict[str, type]:
    if HAVE_VLLM:  # pragma: no cover
        from vllm.model_executor.layers.quantization import QUANTIZATION_METHODS  # noqa: F401
        return {}
    return _QUANT_REGISTRY
