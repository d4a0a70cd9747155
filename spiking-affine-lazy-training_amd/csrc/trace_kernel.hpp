// Arguments and launcher of the trace kernel (trace_kernel.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "salt_device.hpp"

namespace salt {

struct TraceArgs {
  int conv;                               // 1 = conv layer, 0 = FC
  int IC, Hin, Win, K, S, P, H, W, mql;   // conv geometry
  int n_in, n_out;                        // FC
  int n;                                  // neurons
  int steps;                              // columns per neuron
  int sat;                                // saturate (else wrap)
  Quant qz;
  const int32_t* table;
  const void* q;                          // conv (oc, ic, k, k); FC (n_in, n_out)
  int q_bits;
  int L;
  const float* times;
  const int32_t* src;
  const int32_t* n_real;
  int32_t* v_steps;                       // [B][n][steps]
  float* event_ms;                        // [B][n][steps]
  uint8_t* flags;                         // [B][n][steps]: bit 0 spike, bit 1 overflow
};

hipError_t launch_trace(const TraceArgs& a, int B, hipStream_t st);

}  // namespace salt
