"""aneforge_amd: an MI355X-native (gfx950 HIP) rebuild of ANEForge's quantized-decode path,
behind the reference's Python API (aneforge/__init__.py:13-38):

  af.input / af.Tensor / af.sdpa / af.concat / af.select      lazy graph (graph.py)
  af.compile(out, compress=...) -> Model                      kernel lowering (_compile.py)
  af.LlamaConfig / af.LlamaPrefill / af.load_llm / af.rope     decoder on the device (llm.py)
  af.moe (load_gguf, _moe, _topk_gate)                         sparse MoE (moe.py)
  aneforge_amd.speculative.spec_generate                       greedy speculative decoding (speculative.py)

Compute runs in hand-written HIP kernels for gfx950 (libaneforge_hip.so, include/aneforge_hip.h);
PyTorch-ROCm only allocates device memory and provides streams.  There is no CPU fallback."""
__version__ = "0.1.0"

from .graph import Tensor, concat, input, maximum, minimum, sdpa, select  # noqa: F401,E402
from ._compile import (CompressionFallbackWarning, Model, MultiModel, PrecisionWarning,  # noqa: F401,E402
                       compile, compile_multi)
from .llm import (LayerSpec, LlamaConfig, LlamaPrefill, from_pretrained as load_llm, rope,  # noqa: F401,E402
                  rope_tables)
from . import moe as moe  # noqa: F401,E402  (registers the "moe" decode MLP and the Qwen-MoE adapter)
from ._gguf import GGUFView  # noqa: F401,E402

__all__ = ["Tensor", "input", "concat", "select", "maximum", "minimum", "sdpa", "compile", "compile_multi",
           "Model", "MultiModel", "CompressionFallbackWarning", "PrecisionWarning", "LlamaConfig", "LayerSpec",
           "LlamaPrefill", "load_llm", "rope", "rope_tables", "moe", "GGUFView"]
