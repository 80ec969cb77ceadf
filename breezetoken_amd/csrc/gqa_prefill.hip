// Causal GQA prefill attention on gfx950 bf16 MFMA (kernel under construction).
#include "bt_common.h"
#include "bt_kernels.h"

namespace bt {

hipError_t launch_prefill(const PrefillParams& p, int head_dim, hipStream_t stream) {
  (void)p; (void)head_dim; (void)stream;
  return hipErrorNotSupported;
}

}  // namespace bt
