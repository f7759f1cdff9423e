// The key filter's backward for float16 key inputs (the kernel template is in keys_backward.h).
#include "keys_backward.h"

extern "C" int vsp_key_filter_backward_f16(const void* z, const float* history, const float* taps, const void* grad_keys,
                                           void* grad_z, float* grad_taps, float* grad_history, void* workspace,
                                           size_t workspace_bytes, int B, int N, int D, int heads, int K, void* stream) {
  return vsp::key_filter_backward<_Float16>(static_cast<const _Float16*>(z), history, taps,
                                            static_cast<const _Float16*>(grad_keys), static_cast<_Float16*>(grad_z),
                                            grad_taps, grad_history, workspace, workspace_bytes, B, N, D, heads, K,
                                            stream, "vsp_key_filter_backward_f16");
}
