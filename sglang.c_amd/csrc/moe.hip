// moe.hip — routed-expert FFN over device-resident quantized experts.
#include "sglq_dev.hpp"

extern "C" int sglq_moe_forward(sglq_dev *const *gate_up, sglq_dev *const *down, int n_exp,
                                const void *h, int h_dtype, int64_t T, const int32_t *topk_ids,
                                const float *topk_w, int k, float *out, void *stream) {
  (void)gate_up; (void)down; (void)n_exp; (void)h; (void)h_dtype; (void)T; (void)topk_ids;
  (void)topk_w; (void)k; (void)out; (void)stream;
  sglq_log_error("qmoe: not available in this build");
  return -1;
}
