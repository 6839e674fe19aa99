// OneTrans block forward (placeholder until the MFMA kernels land).
#include "pdm_common.h"

using namespace pdm;

extern "C" int64_t pdm_onetrans_block_workspace_size(const pdm_block_desc* desc) {
  (void)desc;
  return 0;
}

extern "C" int pdm_onetrans_block_fwd(const pdm_block_desc* desc, const float* x, const pdm_block_weights* w,
                                      float* y, void* workspace, int64_t workspace_bytes, pdm_stream_t stream) {
  (void)desc; (void)x; (void)w; (void)y; (void)workspace; (void)workspace_bytes; (void)stream;
  set_error("pdm_onetrans_block_fwd: not built yet");
  return PDM_ERR_UNSUPPORTED;
}
