"""Kernel-level entry points with the reference's module layout
(nkilab/kernels/{matmul,norm,attention}.py): the tile constants its callers
read (``TK``, ``TM``, ``TN``, ``T``, ``P``) and the kernel functions under
their names and argument layouts (pre-transposed ``lhsT`` / ``qT`` / ``kT``,
tile-multiple shapes), each running the gfx950 kernel behind ``nkilab.ops``.
The reference runs these through ``nki.simulate(kernel)(...)``; here a call
runs on the GPU directly (``simulate(kernel)`` returns the kernel unchanged,
for code written against that form)."""


def simulate(kernel):
    """The reference's ``nki.simulate(kernel)``: these kernels need no simulator."""
    return kernel
