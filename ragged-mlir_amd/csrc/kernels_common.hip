// Op-independent kernels: counter reset, classification, checked offsets.
#define RG_PROLOGUE_KERNELS
#include "kernels.hpp"
#include "table.hpp"

namespace rg {

const void* kernel_reset() { return (const void*)&k_reset; }
const void* kernel_classify(int offsets_dtype) {
  return offsets_dtype ? (const void*)&k_classify<int64_t> : (const void*)&k_classify<int32_t>;
}
const void* kernel_offsets_init() { return (const void*)&k_offsets_init; }
const void* kernel_offsets_check(int offsets_dtype) {
  return offsets_dtype ? (const void*)&k_offsets_check<int64_t> : (const void*)&k_offsets_check<int32_t>;
}

}  // namespace rg
