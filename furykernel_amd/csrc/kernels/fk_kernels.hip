// fk_kernels.hip — the translation unit of the target's hand-written gfx950
// kernels, compiled once into the code object fk_kernels.hsaco that the
// runtime loads (include/fkrocm.h: fk_module_load).
#include "fk_gemv.h"
#include "fk_rows.h"
#include "fk_misc.h"
#include "fk_step.h"
#include "fk_gemm.h"
#include "fk_prefill.h"
