// Max kernels of every dtype / offsets dtype / geometry.
#include "kernels.hpp"
#include "table.hpp"

namespace rg {

static const KernelSet kMax[2][2][kGeometries] = {
    RG_GEOMETRIES(OP_MAX, int32_t, false),
    RG_GEOMETRIES(OP_MAX, int64_t, false),
};

const KernelSet* kernels_max(int dtype, int offsets_dtype, int geometry) {
  return &kMax[offsets_dtype][dtype][geometry];
}

}  // namespace rg
