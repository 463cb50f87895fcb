"""nkilab for MI355X: the nki-kernel-lab kernel set as hand-written gfx950 HIP.

Public surface (as in the reference package): ``nkilab.ops`` (matmul,
choose_blocks, softmax, rmsnorm, swiglu, attention, ATTENTION_VARIANTS) and
``nkilab.model`` (BlockConfig, RMSNorm, DecoderBlock, nki_forward).  The
kernels live in libnkilab_hip.so next to this file (built by nkilab.build).
"""
__version__ = "0.1.0"
