// The key filter's backward for float32 key inputs (the kernel template is in keys_backward.h).
#include "keys_backward.h"

extern "C" int vsp_key_filter_backward_f32(const float* z, const float* history, const float* taps,
                                           const float* grad_keys, float* grad_z, float* grad_taps,
                                           float* grad_history, void* workspace, size_t workspace_bytes, int B, int N,
                                           int D, int heads, int K, void* stream) {
  return vsp::key_filter_backward<float>(z, history, taps, grad_keys, grad_z, grad_taps, grad_history, workspace,
                                         workspace_bytes, B, N, D, heads, K, stream, "vsp_key_filter_backward_f32");
}
