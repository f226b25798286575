// placeholder until the fused log-prob kernel lands
#include "common.h"
extern "C" size_t dsv41_logprob_workspace_bytes(const dsv41_logprob_desc*) { return 0; }
extern "C" int dsv41_logprob_run(const dsv41_logprob_desc*, void*, size_t, void*) {
  return dsv41::fail(DSV41_E_UNSUPPORTED, "not built yet");
}
