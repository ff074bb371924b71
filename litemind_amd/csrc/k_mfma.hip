// k_mfma.hip -- grouped SwiGLU on MFMA for large token counts (placeholder until
// the fp16 MFMA kernels land; the GEMV path serves every token count meanwhile).
#include "lm_internal.h"

namespace lm {

hipError_t launch_mfma_gateup(const ExpertArgs&, int64_t, hipStream_t) { return hipErrorNotSupported; }
hipError_t launch_mfma_down(const ExpertArgs&, int64_t, hipStream_t) { return hipErrorNotSupported; }

}  // namespace lm
