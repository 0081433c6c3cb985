// pkv_prefill.hip -- chunked-prefill attention over the paged pool (gfx950).
// Not provided yet: pkv_prefill_attention reports PKV_ERR_UNSUPPORTED.
#include "pkv_device.h"
#include "pkv_internal.h"

namespace pkv {

bool prefill_supported(const pkv_pool* p, int n_head) {
  (void)p;
  (void)n_head;
  return false;
}

hipError_t launch_prefill(const pkv_pool* p, int layer, const PrefillArgs& a,
                          hipStream_t stream) {
  (void)p;
  (void)layer;
  (void)a;
  (void)stream;
  return hipErrorNotSupported;
}

}  // namespace pkv
