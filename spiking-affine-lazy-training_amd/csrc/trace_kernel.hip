// Trace mode of the integer forward: every neuron's register after every step of its
// queue, with the step's spike and overflow flags and the time of the event it
// processed -- the (n, steps) trajectories of salt_core/quant/scan.py:83-132
// (run_layer_traced) and salt_core/trace.py:13-55 (LayerForwardTrace, event_ms).
//
// A debug and calibration path, not the hot path: one thread per neuron walks the
// stream's events in order (staged through LDS 256 at a time) and keeps its own queue
// position, so the kernel shares no code with the event-parallel layer kernels and
// serves as an independent restatement of the per-neuron queue.
//
// Columns (steps) per neuron:
//   FC   (steps = L, the input stream length): column j is input event j; columns at or
//        beyond n_real are identity steps (dt = 0, code 0), event_ms = NaN.
//   conv (steps = max_queue_len): the events whose candidate positions include the
//        neuron's, in global order, the first max_queue_len of them; then, when the
//        queue has room, one catch-up column decaying to the last input event's time
//        (salt_core/connectivity/conv.py:102-125) and identity columns after it, all
//        with event_ms = NaN.
#include <hip/hip_runtime.h>

#include <cmath>

#include "salt_device.hpp"
#include "trace_kernel.hpp"

namespace salt {

namespace {

constexpr int kTraceBlock = 256;

// Decay code of a gap (times non-decreasing; the wrap-around difference read unsigned).
__device__ __forceinline__ int32_t trace_decay(const TraceArgs& a, int dt) {
  const uint32_t d = (uint32_t)dt, n = (uint32_t)a.qz.n_table;
  if (d == 0) return 1 << a.qz.fa;  // identity column
  return d <= n ? a.table[d - 1] : 0;
}

__device__ __forceinline__ int32_t trace_vth(const TraceArgs& a, int neuron, int channel) {
  switch (a.qz.vth_kind) {
    case SALT_VTH_SCALAR: return a.qz.vth_scalar;
    case SALT_VTH_PER_CHANNEL: return a.qz.vth[channel];
    case SALT_VTH_PER_NEURON: return a.qz.vth[neuron];
    default: return INT_MAX;  // never fires (registers stay below 2^29)
  }
}

// One queue column: process_event (salt_core/quant/scan.py:22-52) and the outputs.
struct TraceNeuron {
  int32_t v = 0;
  int32_t vth;
  size_t row;  // offset of this neuron's first column

  __device__ void step(const TraceArgs& a, int col, int32_t A, int32_t code, float ms) {
    const int32_t d = decay_mul<false>(v, A, a.qz.fa, a.qz.rc);
    const int32_t u = (int32_t)((uint32_t)d + ((uint32_t)code << a.qz.fV));
    const bool ovf = u < -a.qz.half || u > a.qz.half - 1;
    const int32_t f = a.sat ? min(max(u, -a.qz.half), a.qz.half - 1)
                            : __builtin_amdgcn_sbfe(u, 0, a.qz.wbits);
    const bool fire = f >= vth;
    v = fire ? 0 : f;
    a.v_steps[row + col] = v;
    a.event_ms[row + col] = ms;
    a.flags[row + col] = (uint8_t)((fire ? 1 : 0) | (ovf ? 2 : 0));
  }
};

__global__ void __launch_bounds__(kTraceBlock) trace_kernel(TraceArgs a) {
  __shared__ int32_t st_t[kTraceBlock];
  __shared__ int32_t st_s[kTraceBlock];
  __shared__ float st_f[kTraceBlock];
  const int b = blockIdx.y;
  const int i = blockIdx.x * kTraceBlock + threadIdx.x;
  const bool on = i < a.n;
  const int L = a.L;
  const int nr = a.n_real[b];
  const int n_eff = nr < 0 ? 0 : (nr < L ? nr : L);
  const float* tb = a.times + (size_t)b * L;
  const int32_t* sb = a.src + (size_t)b * L;
  const float nan = __builtin_nanf("");

  TraceNeuron nu;
  nu.row = ((size_t)b * a.n + (on ? i : 0)) * (size_t)a.steps;
  int oc = 0, oy = 0, ox = 0;
  if (a.conv) {
    const int HW = a.H * a.W;
    oc = on ? i / HW : 0;
    const int pos = on ? i - oc * HW : 0;
    oy = pos / a.W;
    ox = pos - oy * a.W;
  }
  nu.vth = on ? trace_vth(a, i, a.conv ? oc : i) : INT_MAX;
  int cnt = 0, t_last = 0;

  for (int j0 = 0; j0 < n_eff; j0 += kTraceBlock) {
    const int m = min(kTraceBlock, n_eff - j0);
    __syncthreads();  // the previous chunk has been consumed
    if (threadIdx.x < m) {
      const float tf = tb[j0 + threadIdx.x];
      st_f[threadIdx.x] = tf;
      st_t[threadIdx.x] = time_ms(tf);
      st_s[threadIdx.x] = sb[j0 + threadIdx.x];
    }
    __syncthreads();
    if (!on) continue;
    for (int e = 0; e < m; ++e) {
      const int t = st_t[e];
      const int s = st_s[e];
      if (!a.conv) {  // FC: every event is this neuron's next column
        const int src = min(max(s, 0), a.n_in - 1);  // memory safety; the host checks ids
        const int32_t code = load_code_bits(a.q, (size_t)src * a.n_out + i, a.q_bits);
        nu.step(a, j0 + e, trace_decay(a, t - t_last), code, st_f[e]);
        t_last = t;
        continue;
      }
      const int hw_in = a.Hin * a.Win;
      const int c = min(max(s / hw_in, 0), a.IC - 1);
      const int rem = s - (s / hw_in) * hw_in;
      const int y = rem / a.Win, x = rem - (rem / a.Win) * a.Win;
      const int ky = y - a.S * oy + a.P, kx = x - a.S * ox + a.P;
      if (ky < 0 || ky >= a.K || kx < 0 || kx >= a.K) continue;
      if (cnt < a.mql) {
        const size_t qi = (((size_t)oc * a.IC + c) * a.K + ky) * a.K + kx;
        nu.step(a, cnt, trace_decay(a, t - t_last), load_code_bits(a.q, qi, a.q_bits), st_f[e]);
        t_last = t;
      }
      ++cnt;  // counted past max_queue_len too: such a queue has no free column
    }
  }
  if (!on) return;
  int col = a.conv ? cnt : n_eff;
  if (a.conv && col < a.steps) {
    // catch-up column: decay to the last input event's time (dt = 0 for an empty queue)
    const int T = n_eff > 0 ? time_ms(tb[n_eff - 1]) : 0;
    nu.step(a, col, trace_decay(a, cnt > 0 ? T - t_last : 0), 0, nan);
    ++col;
  }
  for (; col < a.steps; ++col) nu.step(a, col, trace_decay(a, 0), 0, nan);
}

}  // namespace

hipError_t launch_trace(const TraceArgs& a, int B, hipStream_t st) {
  const dim3 grid((a.n + kTraceBlock - 1) / kTraceBlock, B);
  hipLaunchKernelGGL(trace_kernel, grid, dim3(kTraceBlock), 0, st, a);
  return hipGetLastError();
}

}  // namespace salt
