"""furykernel_amd — FuryKernel's execution target for AMD Instinct MI355X (gfx950).

The pieces, from the bottom:

* ``runtime`` — the C ABI of ``include/fkrocm.h`` (``libfkrocm.so``): device
  context, code-object modules, resident arenas, copies, launches, events and
  graphs.
* ``kernels`` — the launch table of the hand-written gfx950 kernels
  (``fk_kernels.hsaco``).
* ``target`` — ``Rocm``'s caps and backend, the interface FuryKernel's CPU
  target implements (src/FuryKernel/Target.hs, src/FuryKernel/Backend.hs).
* ``program`` — the program layer's graph, builder, gate and planner, the
  host side that turns a model's step into launches.
* ``engine`` — runs a plan's steps on the GPU, its state resident in HBM.

Nothing here computes on the CPU in place of the GPU: without the native
library or a GPU, the runtime raises.
"""

__all__ = ["runtime", "kernels"]
