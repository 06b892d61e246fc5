"""switchyard for MI355X: the Block AttnRes operator on hand-written HIP.

Submodules (imported directly, as in the reference):
  ``switchyard.hip_op``     the operator (autograd + batched), HIP-backed
  ``switchyard.triton_op``  import-compatible alias of the reference's module
  ``switchyard.reference``  DEFAULT_EPS, BlockAttnRes parameters, byte model
  ``switchyard.baselines``  eager PyTorch formulations (comparators)
  ``switchyard.model``      decoder Transformer with a source arena
  ``switchyard.harness``    measurement primitives
"""

__version__ = "0.1.0"
