"""Import-compatible alias of the reference's ``switchyard.triton_op``.

Existing callers write ``from switchyard.triton_op import
block_attn_res_triton`` (reference README.md:132, tests/test_triton_op.py:23-30).
This module keeps those names working; every one of them is the HIP
implementation in :mod:`switchyard.hip_op`. There is no Triton here.
"""

from __future__ import annotations

from .hip_op import (  # noqa: F401
    BlockAttnResHIP,
    _batched_launch,
    _bwd_launch,
    _launch_config,
    bandwidth_probe,
    block_attn_res_batched,
    block_attn_res_hip,
    speed_of_light,
)

#: The reference's names for the same objects.
block_attn_res_triton = block_attn_res_hip
BlockAttnResTriton = BlockAttnResHIP

__all__ = ["block_attn_res_triton", "block_attn_res_batched", "BlockAttnResTriton"]
