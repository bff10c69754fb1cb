// Kernel tables: every compiled specialisation, addressed by
// (op, dtype, offsets dtype, geometry, mask). One translation unit per op
// (inst_sum.hip, inst_max.hip, inst_softmax.hip) instantiates its kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "fused.hpp"
#include "worker.hpp"

namespace rg {

struct KernelSet {
  const void* naive;
  const void* worker;            // classified schedule: wave, block and split classes in one launch
  const void* fused;             // softmax, row mapping: register-resident worker
  const void* fused_f32;         // same, storing f32 logits (scale or mask on bf16 input)
  int vec;                       // elements per vector access
  bool flat;                     // flat mapping (D < vec)
  int rpt;                       // rows per thread of `fused` (0: no fused worker)
  int rpt_f32;                   // rows per thread of `fused_f32`
};

// Rows per thread of the register-resident softmax: 256 bytes of row data
// per thread (64 VGPRs), at most 32 rows.
template <class S, int VEC>
constexpr int fused_rows() {
  return 256 / (VEC * (int)sizeof(S)) > 32 ? 32 : 256 / (VEC * (int)sizeof(S));
}

template <int OP, class T, class OFFT, int VEC, bool FLAT, bool MASK, bool STORE_F32>
constexpr const void* fused_kernel() {
  if constexpr (OP == OP_SOFTMAX && !FLAT && (STORE_F32 || !MASK)) {
    using Store = typename std::conditional<STORE_F32, float, T>::type;
    return (const void*)&k_softmax_fused<T, OFFT, VEC, fused_rows<Store, VEC>(), MASK, STORE_F32>;
  } else {
    return nullptr;
  }
}

template <int OP, class T, int VEC, bool FLAT, bool MASK, bool STORE_F32>
constexpr int fused_rpt() {
  if constexpr (OP == OP_SOFTMAX && !FLAT && (STORE_F32 || !MASK))
    return fused_rows<typename std::conditional<STORE_F32, float, T>::type, VEC>();
  else
    return 0;
}

// Geometry index: f32 -> 0:row1 1:row2 2:row4 3:flat4; bf16 -> 0:row1 1:row2 2:row4 3:row8 4:flat8.
constexpr int kGeometries = 5;

const KernelSet* kernels_sum(int dtype, int offsets_dtype, int geometry);
const KernelSet* kernels_max(int dtype, int offsets_dtype, int geometry);
const KernelSet* kernels_softmax(int dtype, int offsets_dtype, int geometry, bool mask);

// Counter reset, classification and checked-mode kernels (op independent), in kernels_common.hip.
const void* kernel_reset();
const void* kernel_classify(int offsets_dtype);
const void* kernel_offsets_init();
const void* kernel_offsets_check(int offsets_dtype);

}  // namespace rg

#define RG_SET(OP, T, OFFT, VEC, FLAT, MASK)                                              \
  {(const void*)&rg::k_naive<OP, T, OFFT, VEC, FLAT, MASK>,                               \
   (const void*)&rg::k_worker<OP, T, OFFT, VEC, FLAT, MASK>,                              \
   rg::fused_kernel<OP, T, OFFT, VEC, FLAT, MASK, std::is_same<T, float>::value>(),              \
   rg::fused_kernel<OP, T, OFFT, VEC, FLAT, MASK, true>(),                                       \
   VEC, FLAT,                                                                                    \
   rg::fused_rpt<OP, T, VEC, FLAT, MASK, std::is_same<T, float>::value>(),                       \
   rg::fused_rpt<OP, T, VEC, FLAT, MASK, true>()}

// All geometries of one (op, offsets dtype, mask): f32 row then bf16 row.
#define RG_GEOMETRIES(OP, OFFT, MASK)                                                           \
  {{RG_SET(OP, float, OFFT, 1, false, MASK), RG_SET(OP, float, OFFT, 2, false, MASK),          \
    RG_SET(OP, float, OFFT, 4, false, MASK), RG_SET(OP, float, OFFT, 4, true, MASK),           \
    {nullptr, nullptr, nullptr, nullptr, 0, false, 0, 0}},                                      \
   {RG_SET(OP, __bf16, OFFT, 1, false, MASK), RG_SET(OP, __bf16, OFFT, 2, false, MASK),        \
    RG_SET(OP, __bf16, OFFT, 4, false, MASK), RG_SET(OP, __bf16, OFFT, 8, false, MASK),        \
    RG_SET(OP, __bf16, OFFT, 8, true, MASK)}}
