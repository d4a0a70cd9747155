// Event-driven integer FC layer (salt_core/layers/fc.py:84-124 with the queue of
// salt_core/connectivity/fc.py:20-61 and the scan of salt_core/quant/scan.py:22-132).
//
// One wave = one stream x one slice of 64*NPL neurons (neuron = n0 + k*64 + lane);
// registers, extremes and thresholds stay in VGPRs.  A stream's slices are either
// separate work-groups that write spike masks (compacted afterwards), or the waves of one
// work-group (up to kFcMaxWaves) that append to the stream directly: after each chunk the
// waves exchange their per-event spike counts through LDS, so each places its own
// spikes after those of the lower waves -- the (event, neuron) order of the reference.  Every real event updates every
// neuron with the same decay code (the FC queue's dt is the gap to the previous real
// event, the first against t = 0), so the codes of 64 events are looked up at once,
// one per lane, and read back per event with v_readlane.  The event's weight column
// comes from the transposed (n_in, n_out) copy -- from LDS when the slice's columns fit
// (WLDS), else from global memory -- and is loaded 2 to 11 events ahead.
#pragma once

#include <type_traits>

#include "salt_device.hpp"

namespace salt {

constexpr int kFcMaxWaves = 4;  // waves per stream of a directly appending FC layer

// LDS of an FC work-group: the extended decay table (n_table + 2 words), padded to 16
// bytes, then the slice's weights (WLDS) or the merge buffers.
__host__ __device__ inline int fc_lds_table_words(int n_table) { return (n_table + 2 + 3) & ~3; }

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
template <typename QT, int NPL, bool SAT, bool WLDS, bool NOFIRE, bool DIRECT>
__device__ __forceinline__ void fc_events(const FcArgs& a, const QT* wl, const QT* qt,
                                          const int (&col)[NPL], int sw, int n0, int b,
                                          int base, int ne, int tv, int sv, int Aj,
                                          int32_t (&V)[NPL], int32_t (&mn)[NPL],
                                          int32_t (&mx)[NPL], const int32_t (&vth)[NPL],
                                          int& out_base, int32_t* merge) {
  const Quant& qz = a.qz;
  const int fa = qz.fa, fV = qz.fV;
  // The rounding constant in a VGPR for the whole loop: a VALU instruction reads one
  // scalar operand here, and the decay multiply-add's is the event's decay code.
  int rc = qz.rc;
  asm volatile("" : "+v"(rc));
  const int lane = threadIdx.x & (kWave - 1);
  // WLDS: lane e holds the LDS index of its event's weight row, multiplied out once per
  // chunk, so that no scalar instruction waits for a v_readlane in the loop.
  const int rowv = WLDS ? sv * sw : 0;
  // An event's operands, fetched ahead of its step: its decay code and, per neuron, its
  // weight.  Lanes past the slice read a valid weight of the slice (col is clamped) and
  // are never reported; their threshold is unreachable.
  auto load = [&](QT (&q)[NPL], int& A, int e) {  // past the chunk: a harmless reload
    const int ec = min(e, kWave - 1);
    A = rdlane(Aj, ec);
    if (WLDS) {
      const int row = rdlane(rowv, ec);
#pragma unroll
      for (int k = 0; k < NPL; ++k) q[k] = wl[row + col[k]];
    } else {
      const int s_e = rdlane(sv, ec);
      if constexpr (NPL >= 4) {
        // Wide slices: the row base in scalar registers and a 32-bit lane offset, so the
        // load takes the scalar-base form and no 64-bit multiply-add runs per event (the
        // empty asms keep the base scalar and the offset 32-bit; address space 1 keeps
        // the load global): configuration 5 24.4 -> 22.7 ms.  A lone wave (configuration
        // 1) pays for the scalar chain readlane -> multiply -> add on every event
        // instead: 0.231 -> 0.297 ms, so narrow slices keep the vector form.
        typedef const __attribute__((address_space(1))) char gchar;
        typedef const __attribute__((address_space(1))) QT gqt;
        gchar* rowb = (gchar*)(qt + ((size_t)s_e * a.n_out + n0));
        asm volatile("" : "+s"(rowb));
#pragma unroll
        for (int k = 0; k < NPL; ++k) {
          uint32_t ob = (uint32_t)col[k] * (uint32_t)sizeof(QT);
          asm volatile("" : "+v"(ob));
          q[k] = *(gqt*)(rowb + ob);
        }
      } else {
#pragma unroll
        for (int k = 0; k < NPL; ++k) q[k] = qt[(size_t)s_e * a.n_out + n0 + col[k]];
      }
    }
  };
  // DIRECT: lane e of klo/khi[k] collects event e's ballot of the neurons that kept their
  // value (written by v_writelane from the compare's scalar result: no per-lane bit
  // arithmetic in the loop); the chunk's spikes are placed after its events.
  uint32_t klo[NPL], khi[NPL];
#pragma unroll
  for (int k = 0; k < NPL; ++k) klo[k] = khi[k] = ~0u;
  // One event: process_event (salt_core/quant/scan.py:22-52) for every neuron, then its
  // spikes.  LO: the slice has 32 neurons or fewer, so the ballot's low half holds them.
  // FV0: f_V = 0, the weight is added unshifted.
  auto step = [&](int e, const QT (&qc)[NPL], int A, auto lo_only, auto fv0) {
    constexpr bool LO = decltype(lo_only)::value, FV0 = decltype(fv0)::value;
#pragma unroll
    for (int k = 0; k < NPL; ++k) {
      // The decay as one 64-bit multiply-add: configuration 1 0.325 -> 0.269 ms and 5
      // 35.2 -> 32.5 ms against the split 24-bit form.  (Folding the weight into it too,
      // (A*V + c + w*2^f_a) >> f_a, shortens the chain but costs an instruction:
      // measured slower.)
      const int32_t d = decay_mul_wide(V[k], A, fa, rc);
      const uint32_t qw = FV0 ? (uint32_t)(int32_t)qc[k] : ((uint32_t)(int32_t)qc[k] << fV);
      const int32_t u = (int32_t)((uint32_t)d + qw);
      const int32_t f = fit_bits<SAT>(u, qz);
      mn[k] = min(mn[k], u);
      mx[k] = max(mx[k], u);
      if (NOFIRE) {  // no threshold: the write-back is the register's whole chain
        V[k] = f;
        if (DIRECT) continue;
      }
      const bool keep = NOFIRE || f < vth[k];
      if (!NOFIRE) V[k] = keep ? f : 0;
      const uint64_t bal = __ballot(keep);
      if (DIRECT) {
        if (LO) stage_to_lane_lo(klo[k], bal, e);
        else stage_to_lane(klo[k], khi[k], bal, e);
      } else {
        const int w0 = (n0 + k * kWave) >> 5;
        if (lane < 2 && w0 + lane < a.words)
          a.masks[((size_t)b * a.L + base + e) * a.words + w0 + lane] =
              ~(lane ? (uint32_t)(bal >> 32) : (uint32_t)bal);
      }
    }
  };
  // A full chunk of a readout (no threshold, a slice of one word of neurons appending
  // directly): the weights of all 64 events are loaded first, then the 64 updates run
  // unrolled, so the wave waits only on the register's own chain (configuration 3's
  // readout 0.181 -> 0.142 ms).  The same for slices that fire, with the ballots staged
  // at immediate lane indices, measured slower (configuration 1: 0.30 -> 0.33 ms).
  if constexpr (DIRECT && NOFIRE && NPL == 1) {
    if (ne == kWave) {
      int32_t qv[kWave];
#pragma unroll
      for (int i = 0; i < kWave; ++i) {
        if (WLDS) qv[i] = (int32_t)wl[rdlane(rowv, i) + col[0]];
        else qv[i] = (int32_t)qt[(size_t)rdlane(sv, i) * a.n_out + n0 + col[0]];
      }
      // The lone wave of a readout is bound by its instruction count here: the decay as
      // one 64-bit multiply-add and the extremes over pairs of events take it from about
      // 12 to 8 instructions per update (configuration 3's readout 0.106 -> 0.095 ms).
      // (Folding the weight into that multiply-add as well shortens the chain -- 27
      // against 38 clock ticks per update in isolation -- but costs an instruction.)
#pragma unroll
      for (int i = 0; i < kWave; i += 2) {
        const int32_t d0 = decay_mul_wide(V[0], rdlane(Aj, i), fa, rc);
        const int32_t u0 = (int32_t)((uint32_t)d0 + ((uint32_t)qv[i] << fV));
        V[0] = fit_bits<SAT>(u0, qz);
        const int32_t d1 = decay_mul_wide(V[0], rdlane(Aj, i + 1), fa, rc);
        const int32_t u1 = (int32_t)((uint32_t)d1 + ((uint32_t)qv[i + 1] << fV));
        V[0] = fit_bits<SAT>(u1, qz);
        mn[0] = min(mn[0], min(u0, u1));
        mx[0] = max(mx[0], max(u0, u1));
      }
      return;
    }
  }
  // D events per iteration with D operand sets in a ring, each loaded D - 1 events
  // before its use: the loads' latency is covered by D - 1 events of arithmetic and no
  // register has to be copied or widened before its use (either would wait for the
  // load).  Narrow slices have little arithmetic per event and few registers per set,
  // so they look about twelve neuron updates ahead: configuration 1's layer (one neuron
  // per lane, weights from L2) takes 0.254 / 0.264 / 0.239 / 0.232 / 0.230 / 0.237 ms
  // with 3 / 4 / 6 / 9 / 12 / 16 sets.  The scheduling barriers keep each load where it
  // is written: left alone, the compiler sinks a load past the preceding event's
  // arithmetic to just before its own use, and the event then waits for the whole load
  // latency.
  constexpr int D = 12 / NPL > 3 ? 12 / NPL : 3;
  QT q[D][NPL];
  int A[D];
#pragma unroll
  for (int i = 0; i < D; ++i) A[i] = 0;
#pragma unroll
  for (int i = 0; i + 1 < D; ++i) load(q[i], A[i], i);
  int e = 0;
  auto run = [&](auto lo_only, auto fv0) {
    // invariant at the loop head: set i holds event e + i, for i < D - 1
    for (; e + D - 1 < ne; e += D) {
#pragma unroll
      for (int i = 0; i < D; ++i) {
        load(q[(i + D - 1) % D], A[(i + D - 1) % D], e + i + D - 1);
        __builtin_amdgcn_sched_barrier(0);
        step(e + i, q[i], A[i], lo_only, fv0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int i = 0; i + 1 < D; ++i)
      if (e < ne) step(e++, q[i], A[i], lo_only, fv0);
  };
  const bool lo = DIRECT && NPL == 1 && sw <= 32;
  if (fV == 0) {
    if (lo) run(std::true_type{}, std::true_type{});
    else run(std::false_type{}, std::true_type{});
  } else {
    if (lo) run(std::true_type{}, std::false_type{});
    else run(std::false_type{}, std::false_type{});
  }
  if (DIRECT && !NOFIRE) {
    // Lane = the chunk's event: its spikes (neurons ascending) follow those of the
    // chunk's earlier events -- the (event, neuron) order of salt_core/stream.py.
    uint64_t sp[NPL];
    int cnt = 0;
#pragma unroll
    for (int k = 0; k < NPL; ++k) {
      sp[k] = ~(((uint64_t)khi[k] << 32) | klo[k]);
      cnt += __popcll(sp[k]);
    }
    // Several waves per stream: the event's spikes in lower waves (lower neurons) come
    // first.  The counts are double-buffered by chunk parity, so one barrier per chunk
    // orders them: a wave rewrites a buffer only after every wave has passed the next
    // chunk's barrier, i.e. has read it.
    const int wpg = (int)(blockDim.x / kWave);
    int lower = 0, evt = cnt;
    if (wpg > 1) {
      const int wave = (int)(threadIdx.x / kWave);
      int32_t* mc = merge + ((base / kWave) & 1) * (kFcMaxWaves * kWave);
      mc[wave * kWave + lane] = cnt;
      __syncthreads();
      evt = 0;
      for (int w = 0; w < wpg; ++w) {
        const int c = mc[w * kWave + lane];
        evt += c;
        lower += w < wave ? c : 0;
      }
    }
    if (__builtin_expect(__ballot(evt != 0) != 0, 0)) {  // readout layers rarely fire
      const int incl = wave_incl_scan(evt);
      const int total = __builtin_amdgcn_readlane(incl, kWave - 1);
      // Lane = the chunk's event: this wave's spikes of it take places [first, first +
      // cnt) of the chunk's output, which starts at out_base (places from cap on are
      // dropped).
      const int first = incl - evt + lower;
      const int room = a.cap - out_base;
      float* const ot = a.out_t + (size_t)b * a.cap + out_base;
      int32_t* const os = a.out_s + (size_t)b * a.cap + out_base;
      if (total > 2 * kWave) {
        // Dense chunk: event by event with lane = neuron, so each store writes one run of
        // consecutive entries (whole cache lines from one wave in quick succession)
        // instead of one entry in each of 64 runs.  Measured on configuration 5 (~180
        // spikes per event): 63.7 -> 42.0 ms, writes 110 -> 70 GB for 66 GB of entries.
        // Stores address the uniform stream bases plus a 32-bit byte offset (the
        // scalar-base form of the store); the capacity test only in the event that
        // reaches it.
        const int te_bits = __float_as_int(ms_time(tv));
        char* const otb = reinterpret_cast<char*>(ot);
        char* const osb = reinterpret_cast<char*>(os);
        auto place = [&](int e, int at, auto check) {
          constexpr bool kCheck = decltype(check)::value;
          // the event's time in a VGPR once, not moved there again for every store
          float te = __int_as_float(__builtin_amdgcn_readlane(te_bits, e));
          asm volatile("" : "+v"(te));
#pragma unroll
          for (int k = 0; k < NPL; ++k) {
            const uint64_t m =
                ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(sp[k] >> 32), e) << 32) |
                (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)sp[k], e);
            const uint32_t r = (uint32_t)at + __builtin_amdgcn_mbcnt_hi(
                                   (uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
            // The lane's own bit of the uniform mask: the mask itself becomes the
            // execution mask (no per-lane shift, and or compare).
            if (__builtin_amdgcn_inverse_ballot_w64(m) && (!kCheck || (int)r < room)) {
              *reinterpret_cast<float*>(otb + (r << 2)) = te;
              *reinterpret_cast<int32_t*>(osb + (r << 2)) = n0 + k * kWave + lane;
            }
            at += __popcll(m);
          }
        };
        for (uint64_t evs = __ballot(cnt > 0); evs; evs &= evs - 1) {
          const int e = __builtin_ctzll(evs);
          const int at = __builtin_amdgcn_readlane(first, e);
          if (at >= room) break;  // so do the later events'
          if (at + __builtin_amdgcn_readlane(cnt, e) <= room) place(e, at, std::false_type{});
          else place(e, at, std::true_type{});
        }
      } else {
        // Sparse chunk: each lane writes its event's run (a few stores in all).
        const float te = ms_time(tv);
        int pos = first;
#pragma unroll
        for (int k = 0; k < NPL; ++k)
          for (uint64_t bits = sp[k]; bits; bits &= bits - 1) {
            if (pos < room) {
              ot[pos] = te;
              os[pos] = n0 + k * kWave + __builtin_ctzll(bits);
            }
            ++pos;
          }
      }
      out_base += total;
    }
  }
}

// NOFIRE: the layer has no threshold (v_th None: a readout), so nothing fires, no spike
// is staged or placed, and the register's chain per event ends at the write-back.
template <typename QT, int NPL, bool SAT, bool WLDS, bool NOFIRE = false>
__global__ void __launch_bounds__(kFcMaxWaves * kWave) fc_layer_kernel(FcArgs a) {
  extern __shared__ int32_t dyn[];
  const int lane = threadIdx.x & (kWave - 1);
  // wide slices: the wave index (so n0) provably uniform, for the scalar weight-row base
  const int wave = NPL >= 4 ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave))
                            : (int)(threadIdx.x / kWave);
  const int wpg = (int)(blockDim.x / kWave);
  const int b = blockIdx.y;
  const int n0 = (blockIdx.x * wpg + wave) * (kWave * NPL);
  const int sw = min(kWave * NPL, a.n_out - n0);  // neurons in this slice
  const Quant& qz = a.qz;
  int32_t* ext = dyn;
  // after the table, at 16 bytes (fc_lds_table_words)
  QT* wl = reinterpret_cast<QT*>(dyn + fc_lds_table_words(qz.n_table));
  // several waves per stream (never with WLDS): per-event spike counts, two chunk
  // buffers of kFcMaxWaves x 64, then the waves' extremes
  int32_t* merge = dyn + fc_lds_table_words(qz.n_table);
  int32_t* red = merge + 2 * kFcMaxWaves * kWave;
  const QT* qt = static_cast<const QT*>(a.qt);
  load_ext_table(ext, a.table, qz.n_table, qz.fa, (int)threadIdx.x, (int)blockDim.x);
  if (WLDS) {
    const int n = a.n_in * sw;
    if (sw == a.n_out && ((uintptr_t)qt & 15) == 0) {
      // The slice is the whole layer, so its weights are one block: 16-byte copies
      // (a readout's 15 KB in a few microseconds, against 31 element by element).
      const int nbytes = n * (int)sizeof(QT), n16 = nbytes >> 4;
      const uint4* s16 = reinterpret_cast<const uint4*>(qt);
      uint4* d16 = reinterpret_cast<uint4*>(wl);
#pragma unroll 8
      for (int i = lane; i < n16; i += kWave) d16[i] = s16[i];
      for (int i = (n16 << 4) + lane; i < nbytes; i += kWave)
        reinterpret_cast<char*>(wl)[i] = reinterpret_cast<const char*>(qt)[i];
    } else {
      const float rsw = 1.0f / (float)sw;  // n < 2^22: the LDS holds the slice
      for (int i = lane; i < n; i += kWave) {
        const int r = div_small(i, sw, rsw);
        wl[i] = qt[(size_t)r * a.n_out + n0 + (i - r * sw)];
      }
    }
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
      fc_events<QT, NPL, SAT, WLDS, NOFIRE, true>(a, wl, qt, col, sw, n0, b, base, ne, tv,
                                                       sv, Aj,
                                               V, mn, mx, vth, out_base, merge);
    else
      fc_events<QT, NPL, SAT, WLDS, NOFIRE, false>(a, wl, qt, col, sw, n0, b, base, ne, tv,
                                                        sv,
                                                Aj, V, mn, mx, vth, out_base, merge);
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
  if (a.direct && wpg > 1) {  // the stream's extremes over its waves
    if (lane == 0) {
      red[2 * wave] = vmin_l;
      red[2 * wave + 1] = vmax_l;
    }
    __syncthreads();
    for (int w = 0; w < wpg; ++w) {
      vmin_l = min(vmin_l, red[2 * w]);
      vmax_l = max(vmax_l, red[2 * w + 1]);
    }
  }
  const int ovf = (vmin_l < -qz.half || vmax_l > qz.half - 1) ? 1 : 0;
  if (a.direct) {
    if (threadIdx.x == 0) {
      a.out_n[b] = out_base;
      a.stats[b * 4 + 0] = vmin_l;
      a.stats[b * 4 + 1] = vmax_l;
      a.stats[b * 4 + 2] = 0;
      a.stats[b * 4 + 3] = ovf;
    }
    if (a.fill_pads)
      for (int i = min(out_base, a.cap) + (int)threadIdx.x; i < a.cap; i += (int)blockDim.x) {
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
