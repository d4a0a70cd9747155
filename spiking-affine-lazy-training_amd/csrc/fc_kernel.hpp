// Event-driven integer FC layer (salt_core/layers/fc.py:84-124 with the queue of
// salt_core/connectivity/fc.py:20-61 and the scan of salt_core/quant/scan.py:22-132).
//
// One wave = one stream x one slice of 64*NPL neurons (neuron = n0 + k*64 + lane);
// registers, extremes and thresholds stay in VGPRs.  Every real event updates every
// neuron with the same decay code (the FC queue's dt is the gap to the previous real
// event, the first against t = 0), so the codes of 64 events are looked up at once,
// one per lane, and read back per event with v_readlane.  The event's weight column
// comes from the transposed (n_in, n_out) copy -- from LDS when the slice's columns fit
// (WLDS), else from global memory -- and is loaded one event ahead.
#pragma once

#include "salt_device.hpp"

namespace salt {

struct FcArgs {
  int n_in, n_out, words;  // words: 32-bit spike-mask words per event (sliced layers)
  Quant qz;
  const int32_t* table;
  const void* qt;          // (n_in, n_out)
  int q_bits;
  int L;
  const float* times;
  const int32_t* src;
  const int32_t* n_real;
  int cap, fill_pads, direct;
  float* out_t;
  int32_t* out_s;
  int32_t* out_n;
  int32_t* v_final;
  int32_t* v_min;
  int32_t* v_max;
  int32_t* stats;
  uint32_t* masks;
};

// The events of one chunk (one per lane of tv/sv, ne of them) with their decay codes
// Aj.  DIRECT: the slice is the whole layer and appends spikes to the output stream;
// otherwise it writes the chunk's spike-mask words.
template <typename QT, int NPL, bool F24, bool SAT, bool WLDS, bool DIRECT>
__device__ __forceinline__ void fc_events(const FcArgs& a, const QT* wl, const QT* qt,
                                          const int (&col)[NPL], int sw, int n0, int b,
                                          int base, int ne, int tv, int sv, int Aj,
                                          int32_t (&V)[NPL], int32_t (&mn)[NPL],
                                          int32_t (&mx)[NPL], const int32_t (&vth)[NPL],
                                          int& out_base) {
  const Quant& qz = a.qz;
  const int fa = qz.fa, rc = qz.rc, fV = qz.fV;
  const int lane = threadIdx.x;
  // Lanes past the slice read a valid code of the slice (col is clamped) and are never
  // reported; their threshold is unreachable.
  auto column = [&](int s, int k) -> QT {
    return WLDS ? wl[s * sw + col[k]] : qt[(size_t)s * a.n_out + n0 + col[k]];
  };
  // DIRECT: bit e & 31 of fired[h][k] (h = e / 32) records that this lane's neuron k
  // fired at the chunk's event e -- vector operations only, so that the event loop has
  // no branch on the compare -- and the chunk's spikes are appended after its events.
  uint32_t fired[2][NPL];
#pragma unroll
  for (int k = 0; k < NPL; ++k) fired[0][k] = fired[1][k] = 0;
  // One event: process_event (salt_core/quant/scan.py:22-52) for every neuron, then its
  // spikes (DIRECT: recorded in fired[h]; else the chunk's spike-mask words).
  auto step = [&](int e, const QT (&qc)[NPL], uint32_t (&fh)[NPL]) {
    const int A = rdlane(Aj, e);
#pragma unroll
    for (int k = 0; k < NPL; ++k) {
      const int32_t d = decay_mul<F24>(V[k], A, fa, rc);
      const int32_t u = (int32_t)((uint32_t)d + ((uint32_t)(int32_t)qc[k] << fV));
      const int32_t f = fit_bits<SAT>(u, qz);
      const bool fire = f >= vth[k];
      V[k] = fire ? 0 : f;
      mn[k] = min(mn[k], u);
      mx[k] = max(mx[k], u);
      if (DIRECT) {
        fh[k] |= fire ? (1u << (e & 31)) : 0u;
      } else {
        const uint64_t bal = __ballot(fire);
        const int w0 = (n0 + k * kWave) >> 5;
        if (lane < 2 && w0 + lane < a.words)
          a.masks[((size_t)b * a.L + base + e) * a.words + w0 + lane] =
              lane ? (uint32_t)(bal >> 32) : (uint32_t)bal;
      }
    }
  };
  auto load = [&](QT (&q)[NPL], int e) {  // past the chunk: a harmless reload
    const int s_e = rdlane(sv, min(e, kWave - 1));
#pragma unroll
    for (int k = 0; k < NPL; ++k) q[k] = column(s_e, k);
  };
  // Two events per iteration with two column registers, each loaded one event before its
  // use: the loads' latency is covered by an event of arithmetic and no register has to
  // be copied or widened before its use (either would wait for the load).
  QT qa[NPL], qb[NPL];
  load(qa, 0);
  int e = 0;
  // events [e, end) recording into fh; end is even unless it is ne
  auto run = [&](int end, uint32_t (&fh)[NPL]) {
    for (; e + 1 < end; e += 2) {
      load(qb, e + 1);
      step(e, qa, fh);
      load(qa, e + 2);
      step(e + 1, qb, fh);
    }
    if (e < end) step(e++, qa, fh);
  };
  run(min(ne, 32), fired[0]);
  run(ne, fired[1]);
  if (DIRECT) {
    uint32_t any = 0;
#pragma unroll
    for (int k = 0; k < NPL; ++k) any |= fired[0][k] | fired[1][k];
    if (__builtin_expect(__ballot(any != 0) != 0, 0)) {  // readout layers rarely fire
      // (event, neuron) order: per event, the slice's neurons in ascending order
      for (int e2 = 0; e2 < ne; ++e2) {
        const int h = e2 >> 5, sh = e2 & 31;
        // read with every lane active: a lane's VGPR value is only kept for the lanes
        // that use it, so a read of another lane inside the branch below may see a reuse
        const float te = (float)rdlane(tv, e2);
#pragma unroll
        for (int k = 0; k < NPL; ++k) {
          const bool f = ((h ? fired[1][k] : fired[0][k]) >> sh) & 1u;
          const uint64_t bal = __ballot(f);
          if (bal == 0) continue;
          if (f) {
            const int idx = out_base + lanes_below(bal);
            if (idx < a.cap) {
              a.out_t[(size_t)b * a.cap + idx] = te;
              a.out_s[(size_t)b * a.cap + idx] = n0 + k * kWave + lane;
            }
          }
          out_base += __popcll(bal);
        }
      }
    }
  }
}

template <typename QT, int NPL, bool F24, bool SAT, bool WLDS>
__global__ void __launch_bounds__(64) fc_layer_kernel(FcArgs a) {
  extern __shared__ int32_t dyn[];
  const int lane = threadIdx.x;
  const int b = blockIdx.y;
  const int n0 = blockIdx.x * (kWave * NPL);
  const int sw = min(kWave * NPL, a.n_out - n0);  // neurons in this slice
  const Quant& qz = a.qz;
  int32_t* ext = dyn;
  QT* wl = reinterpret_cast<QT*>(dyn + (qz.n_table + 2));
  const QT* qt = static_cast<const QT*>(a.qt);
  load_ext_table(ext, a.table, qz.n_table, qz.fa, lane, kWave);
  if (WLDS)
    for (int i = lane; i < a.n_in * sw; i += kWave) {
      const int r = i / sw;
      wl[i] = qt[(size_t)r * a.n_out + n0 + (i - r * sw)];
    }
  __syncthreads();

  int32_t V[NPL], mn[NPL], mx[NPL], vth[NPL];
  int col[NPL];
  bool nv[NPL];
#pragma unroll
  for (int k = 0; k < NPL; ++k) {
    const int n = n0 + k * kWave + lane;
    nv[k] = n < a.n_out;
    col[k] = min(k * kWave + lane, sw - 1);
    V[k] = 0;
    mn[k] = 0;
    mx[k] = 0;
    int t = INT_MAX;  // no threshold / no neuron: never fires
    if (nv[k]) {
      if (qz.vth_kind == SALT_VTH_SCALAR) t = qz.vth_scalar;
      else if (qz.vth_kind != SALT_VTH_NONE) t = qz.vth[n];
    }
    vth[k] = t;
  }
  const int ntab = qz.n_table;
  const int L = a.L;
  const int nr = a.n_real[b];
  const int n_eff = nr < 0 ? 0 : (nr < L ? nr : L);
  const float* tb = a.times + (size_t)b * L;
  const int32_t* sb = a.src + (size_t)b * L;
  int t_prev = 0;  // the first event is compared with t = 0 (connectivity/fc.py:30)
  int out_base = 0;

  // The next chunk's events are loaded a chunk ahead and converted only when their
  // chunk starts, so the loads' latency is covered by a chunk of work.
  // Loads use an index clamped into the stream (entries past n_eff are never used).
  float t_n = 0.0f;
  int s_n = 0;
  if (n_eff > 0) { t_n = tb[min(lane, n_eff - 1)]; s_n = sb[min(lane, n_eff - 1)]; }

  for (int base = 0; base < n_eff; base += kWave) {
    const int tv = time_ms(t_n), sv = min(max(s_n, 0), a.n_in - 1);
    {
      const int j2 = min(base + kWave + lane, n_eff - 1);
      t_n = tb[j2];
      s_n = sb[j2];
    }
    const int ne = min(kWave, n_eff - base);
    // Decay codes of the chunk's events (salt_core/quant/codes.py:87-105).
    int tp = __shfl_up(tv, 1);
    if (lane == 0) tp = t_prev;
    const int Aj = ext[decay_slot(tv - tp, ntab)];
    t_prev = rdlane(tv, ne - 1);
    if (a.direct)
      fc_events<QT, NPL, F24, SAT, WLDS, true>(a, wl, qt, col, sw, n0, b, base, ne, tv, sv, Aj,
                                               V, mn, mx, vth, out_base);
    else
      fc_events<QT, NPL, F24, SAT, WLDS, false>(a, wl, qt, col, sw, n0, b, base, ne, tv, sv,
                                                Aj, V, mn, mx, vth, out_base);
  }
  // Pad columns (j >= n_real) are identity with code 0 (connectivity/fc.py:32, :60-61):
  // their value before write-back is the final register.
  int vmin_l = 0, vmax_l = 0;
#pragma unroll
  for (int k = 0; k < NPL; ++k) {
    if (!nv[k]) continue;
    if (n_eff < L) {
      mn[k] = min(mn[k], V[k]);
      mx[k] = max(mx[k], V[k]);
    }
    vmin_l = min(vmin_l, mn[k]);
    vmax_l = max(vmax_l, mx[k]);
    const size_t ng = (size_t)b * a.n_out + n0 + k * kWave + lane;
    if (a.v_final) a.v_final[ng] = V[k];
    if (a.v_min) a.v_min[ng] = mn[k];
    if (a.v_max) a.v_max[ng] = mx[k];
  }
  vmin_l = wave_min(vmin_l);
  vmax_l = wave_max(vmax_l);
  const int ovf = (vmin_l < -qz.half || vmax_l > qz.half - 1) ? 1 : 0;
  if (a.direct) {
    if (lane == 0) {
      a.out_n[b] = out_base;
      a.stats[b * 4 + 0] = vmin_l;
      a.stats[b * 4 + 1] = vmax_l;
      a.stats[b * 4 + 2] = 0;
      a.stats[b * 4 + 3] = ovf;
    }
    if (a.fill_pads)
      for (int i = min(out_base, a.cap) + lane; i < a.cap; i += kWave) {
        a.out_t[(size_t)b * a.cap + i] = kPadTime;
        a.out_s[(size_t)b * a.cap + i] = 0;
      }
  } else if (lane == 0) {
    atomicMin(&a.stats[b * 4 + 0], vmin_l);
    atomicMax(&a.stats[b * 4 + 1], vmax_l);
    atomicOr(&a.stats[b * 4 + 3], ovf);
  }
}

}  // namespace salt
