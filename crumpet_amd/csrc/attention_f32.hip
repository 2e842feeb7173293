// f32 instantiations of the fused window attention kernel (attention_kernel.h).
#include "attention_kernel.h"

namespace crumpet {
namespace attn {

void launch_f32(const Params& p, int NT, int kmask, hipStream_t s) { launch<float>(p, NT, kmask, s); }

}  // namespace attn
}  // namespace crumpet
