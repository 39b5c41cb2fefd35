// scratch.h — the per-device scratch array used by
// tca_program_launch_noalloc (defined in scratch.hip).
#ifndef TCA_RT_SCRATCH_H_
#define TCA_RT_SCRATCH_H_

#include <hip/hip_runtime.h>

#include <cstddef>

namespace tca {
namespace rt {

// Size of the array on every device: the most workspace (HBM locals plus the
// partials of split and column reductions) one allocation-free launch may use.
constexpr size_t kScratchBytes = size_t{32} << 20;

// Takes the array's device address on `device`, which must be current.
// Idempotent; called by tca_rt_init.
hipError_t ScratchInit(int device);
// The address ScratchInit took for `device`, or nullptr before it ran.
void* ScratchPtr(int device);

}  // namespace rt
}  // namespace tca

#endif  // TCA_RT_SCRATCH_H_
