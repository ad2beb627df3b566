// fp32 instantiation of the backward kernels.  Built without the VGPR-form
// MFMA option: fp32 operand fragments take twice the registers of fp16, so the
// accumulators (only ever accumulated and stored) live in AGPRs.
#include "capi_internal.h"
#include "train_kernels.h"

namespace fa {
namespace train {

void backward_fp32(const TrainParams& p, bool vec_ok, hipStream_t st) { launch_backward<float>(p, vec_ok, st); }

}  // namespace train
}  // namespace fa
