// Build identification and host-side self-test hooks of the C-ABI library.
#include "spmla_common.h"

extern "C" const char* spmla_version(void) {
  return "spmla-gfx950 0.2 (Row656/Row576; bf16 QK + fp16 PV MFMA; exact radix top-k)";
}

// The e4m3fn encoder the kernels compile (spmla_common.h), run on the host: lets the CPU test suite check it
// against torch's float8_e4m3fn conversion without a GPU.
extern "C" void spmla_host_e4m3_encode(const float* x, uint8_t* out, long long n) {
  for (long long i = 0; i < n; ++i) out[i] = spmla::e4m3_rne(x[i]);
}
