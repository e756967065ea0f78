// Paged prefill / chunked-prefill attention on MFMA (tuned shapes). Until the MFMA
// kernel covers a shape, launch_prefill_attention reports PKV_EUNSUPPORTED and the
// entry point routes the batch to the generic kernel.
#include "attention.h"

namespace pkv {

int launch_prefill_attention(const AttnParams& p, int dtype, hipStream_t stream) {
    (void)p;
    (void)dtype;
    (void)stream;
    return PKV_EUNSUPPORTED;
}

}  // namespace pkv
