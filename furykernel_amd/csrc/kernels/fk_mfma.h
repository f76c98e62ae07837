// fk_mfma.h — what the matrix-core kernels share: the operand vector types of
// the gfx950 v_mfma_f32_*_f16 builtins, raw buffer descriptors, and the
// binary32 -> binary16 conversion of their f16 outputs.
#pragma once

#include "fk_common.h"

typedef _Float16 fk_half8 __attribute__((ext_vector_type(8)));
typedef float fk_float4v __attribute__((ext_vector_type(4)));
typedef float fk_float16v __attribute__((ext_vector_type(16)));

namespace fk {

// Eight f16 operands, as the builtin takes them or as 16 bytes of memory.
union Half8 {
  fk_half8 h;
  uint4 u;
};

// A raw buffer over [base, base + bytes): loads past its end read zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer(const void *base, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0,
                                           (int)(uint32_t)(bytes < 0xffffffffu ? bytes : 0xffffffffu), 0x00020000);
}

// binary32 -> binary16, to nearest even (v_cvt_f16_f32).
__device__ __forceinline__ uint16_t to_f16(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }

}  // namespace fk
