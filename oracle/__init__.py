"""CPU restatement of the reference's W8A8 decoder datapath: TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg, as
the checker of the HIP path (and as the timed CPU baseline). The product
(torch2riscv-accelerator_amd/) never imports, links or runs anything here.

numerics.py  fp32 with flush-to-zero, the SFU, and DeviceModel's vector primitives
model.py     the decoder (DeviceModel generalised to GQA / QK-norm / MoE), prefill
"""
from . import numerics  # noqa: F401
from .model import OracleModel, greedy  # noqa: F401
