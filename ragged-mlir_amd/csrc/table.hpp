// Kernel tables: every compiled specialisation, addressed by
// (op, dtype, offsets dtype, geometry, mask). One translation unit per op
// (inst_sum.hip, inst_max.hip, inst_softmax.hip) instantiates its kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace rg {

struct KernelSet {
  const void* naive;
  const void* wave;
  const void* block;
  const void* split_partial;
  const void* split_combine;
  const void* split_normalize;   // softmax only
  int vec;                       // elements per vector access
  bool flat;                     // flat mapping (D < vec)
};

// Geometry index: f32 -> 0:row1 1:row2 2:row4 3:flat4; bf16 -> 0:row1 1:row2 2:row4 3:row8 4:flat8.
constexpr int kGeometries = 5;

const KernelSet* kernels_sum(int dtype, int offsets_dtype, int geometry);
const KernelSet* kernels_max(int dtype, int offsets_dtype, int geometry);
const KernelSet* kernels_softmax(int dtype, int offsets_dtype, int geometry, bool mask);

// Prologue and checked-mode kernels (op independent), in kernels_common.hip.
const void* kernel_init();
const void* kernel_classify(int offsets_dtype);
const void* kernel_offsets_init();
const void* kernel_offsets_check(int offsets_dtype);

}  // namespace rg

#define RG_SET(OP, T, OFFT, VEC, FLAT, MASK)                                              \
  {(const void*)&rg::k_naive<OP, T, OFFT, VEC, FLAT, MASK>,                               \
   (const void*)&rg::k_wave<OP, T, OFFT, VEC, FLAT, MASK>,                                \
   (const void*)&rg::k_block<OP, T, OFFT, VEC, FLAT, MASK>,                               \
   (const void*)&rg::k_split_partial<OP, T, OFFT, VEC, FLAT, MASK>,                       \
   (const void*)&rg::k_split_combine<OP, T, OFFT, VEC, FLAT, MASK>,                       \
   OP == rg::OP_SOFTMAX ? (const void*)&rg::k_split_normalize<OP, T, OFFT, VEC, FLAT, MASK> : nullptr, \
   VEC, FLAT}

// All geometries of one (op, offsets dtype, mask): f32 row then bf16 row.
#define RG_GEOMETRIES(OP, OFFT, MASK)                                                           \
  {{RG_SET(OP, float, OFFT, 1, false, MASK), RG_SET(OP, float, OFFT, 2, false, MASK),          \
    RG_SET(OP, float, OFFT, 4, false, MASK), RG_SET(OP, float, OFFT, 4, true, MASK),           \
    {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0, false}},                          \
   {RG_SET(OP, __bf16, OFFT, 1, false, MASK), RG_SET(OP, __bf16, OFFT, 2, false, MASK),        \
    RG_SET(OP, __bf16, OFFT, 4, false, MASK), RG_SET(OP, __bf16, OFFT, 8, false, MASK),        \
    RG_SET(OP, __bf16, OFFT, 8, true, MASK)}}
