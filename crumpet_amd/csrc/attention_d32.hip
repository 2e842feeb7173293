// Head-dim-32 instantiations of the fused window attention kernel
// (attention_kernel.h): fp16 and bf16.
#include "attention_kernel.h"

namespace crumpet {
namespace attn {

void launch_d32(const Params& p, int NT, int kmask, int32_t dtype, hipStream_t s) {
    if (dtype == CRUMPET_DTYPE_F16)
        launch32<_Float16>(p, NT, kmask, s);
    else
        launch32<__bf16>(p, NT, kmask, s);
}

}  // namespace attn
}  // namespace crumpet
