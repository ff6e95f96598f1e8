// Instantiations of the bwd scan kernels with fp32 atomics, fp32 activations
// (see mhs_instances.hpp).
#include "mhs_instances.hpp"

namespace mhs {
MHS_FOR_PLANS(MHS_BWD_ATOM_INST, , 4)
}  // namespace mhs
