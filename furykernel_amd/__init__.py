"""furykernel_amd — FuryKernel's execution target for AMD Instinct MI355X (gfx950).

The pieces, from the bottom:

* ``runtime`` — the C ABI of ``include/fkrocm.h`` (``libfkrocm.so``): device
  context, code-object modules, resident arenas, copies, launches, events,
  graphs, the kernels' manifest and ABI hashes, native launch tables, and the
  one-call decode attention of ``include/fkrocm_ops.h``.
* ``kernels`` — the launch table of the hand-written gfx950 kernels
  (``fk_kernels.hsaco``, ``fk_attend.hsaco``) and their launchers.
* ``manifest`` — each kernel's manifest as the reference's JSON.
* ``program`` — the program layer's graph, builder, gate and planner, the
  host side that turns a model's step into launches.
* ``lower`` / ``prefill`` — a plan's steps as launches of the kernels (steps of
  one row, and of many rows on the matrix cores).
* ``engine`` — runs a plan's steps on the GPU, its state resident in HBM;
  ``decode`` and ``prefill`` hold a session over it.
* ``ir`` — the kernel IR, its builder and gate, and the MI355X backend that
  lowers checked kernels to HIP compiled at run time by hipRTC (the
  reference's ``Backend``), with their launcher.
* ``variant``, ``selection``, ``tuning`` — the GEMV families' variant spaces,
  the committed selections and the tuner that writes them.

Nothing here computes on the CPU in place of the GPU: without the native
library or a GPU, the runtime raises.
"""

__all__ = ["runtime", "kernels"]
