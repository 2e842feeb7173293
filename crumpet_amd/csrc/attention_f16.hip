// f16 instantiations of the fused window attention kernel (attention_kernel.h).
#include "attention_kernel.h"

namespace crumpet {
namespace attn {

void launch_f16(const Params& p, int NT, int kmask, hipStream_t s) { launch<_Float16>(p, NT, kmask, s); }

}  // namespace attn
}  // namespace crumpet
