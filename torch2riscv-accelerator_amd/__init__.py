"""MI355X-native W8A8 decoder datapath (drop-in backend for the reference's llm/runtime.py path).

Import it as `t2r_amd` (the shim t2r_amd.py at the repository root loads this directory).

config   model configurations (the five measured shapes, tiny test models)
weights  host-side model data: synthetic weights, W8A8 quantisation, RoPE tables, KV constants
abi      ctypes binding of the C-ABI library libt2r.so (include/t2r.h)
ops      op-level calls (one HIP launch sequence per reference op)
model    DeviceModel: the model resident on one GPU, decode steps and prefill
runtime  LlamaDevice / Sampler: the llm/runtime.py API
"""
from . import config  # noqa: F401
from .config import ModelConfig  # noqa: F401
