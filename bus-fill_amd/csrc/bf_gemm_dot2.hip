// Small-batch GEMM family on v_dot2_f32_f16 (filled in after the MFMA path).
#include "bf_device.h"
#include "bf_launch.h"

namespace bf {

bool dot2_supports(const GemmArgs&) { return false; }

hipError_t gemm_dot2(const GemmArgs&, hipStream_t) { return hipErrorNotSupported; }

}  // namespace bf
