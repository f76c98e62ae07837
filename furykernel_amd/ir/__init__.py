"""The kernel IR and the MI355X target's backend (src/FuryKernel/IR.hs,
Build.hs, Abi.hs, Backend.hs): ``ir`` the IR and its text form, ``build``
the builder kernels are written with, ``gate`` the checks a lowering relies
on, ``abi`` a kernel's ABI and hash, ``reduce`` and ``tile`` the reference's
library of reductions and GEMM tiles, ``rocm`` the backend that lowers
checked kernels to HIP for gfx950, ``runtime`` the hipRTC compile and the
launches of a lowered unit."""
