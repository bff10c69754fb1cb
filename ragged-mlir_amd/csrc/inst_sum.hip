// Sum kernels of every dtype / offsets dtype / geometry.
#include "kernels.hpp"
#include "table.hpp"

namespace rg {

static const KernelSet kSum[2][2][kGeometries] = {
    RG_GEOMETRIES(OP_SUM, int32_t, false),
    RG_GEOMETRIES(OP_SUM, int64_t, false),
};

// Indexed [offsets dtype][dtype][geometry].
const KernelSet* kernels_sum(int dtype, int offsets_dtype, int geometry) {
  return &kSum[offsets_dtype][dtype][geometry];
}

}  // namespace rg
