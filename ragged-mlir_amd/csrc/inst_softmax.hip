// Softmax kernels of every dtype / offsets dtype / geometry, with and without
// the additive f32 mask.
#include "kernels.hpp"
#include "table.hpp"

namespace rg {

static const KernelSet kSoftmax[2][2][2][kGeometries] = {
    {RG_GEOMETRIES(OP_SOFTMAX, int32_t, false), RG_GEOMETRIES(OP_SOFTMAX, int64_t, false)},
    {RG_GEOMETRIES(OP_SOFTMAX, int32_t, true), RG_GEOMETRIES(OP_SOFTMAX, int64_t, true)},
};

const KernelSet* kernels_softmax(int dtype, int offsets_dtype, int geometry, bool mask) {
  return &kSoftmax[mask ? 1 : 0][offsets_dtype][dtype][geometry];
}

}  // namespace rg
