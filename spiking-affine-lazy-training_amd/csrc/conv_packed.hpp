// Event-driven integer conv layer, packed lanes (salt_core/layers/conv.py:124-149 with
// the queue of salt_core/connectivity/conv.py:15-225 and the scan of
// salt_core/quant/scan.py:22-132), for layers whose output plane fits in LDS.
//
// Candidate classes.  An input event at (c, y, x) reaches the output positions of a
// rectangle: rows [max(oy0, 0), min(floor((y+P)/S), H-1)], columns likewise, inside the
// NC x NC grid of candidates starting at (oy0, ox0) = (ceil((y+P-K+1)/S), ...).  Its
// class is the rectangle's shape h x w (1 <= h, w <= NC).  A wave owns Gw output
// channels; for a class of n = h*w candidates it updates G channels per iteration in
// I = ceil(Gw / G) iterations, G = ceil(Gw / I) with I the fewest iterations of at most
// 64 / n channels.  In every iteration lane l < G*n is (channel slot l / n, candidate
// l % n), candidates in row-major order, so a wave instruction carries real updates only,
// apart from the lanes past G*n and the slots past Gw of the last iteration.  Those work
// on zero planes that no neuron owns (zero registers, zero codes, unreachable
// thresholds): U = 0, no spike, neutral for the extremes.  (The lane constants that
// place every lane -- register, code and time-entry offsets and the per-iteration
// strides -- are tables in LDS, one row per class, built at the start.)
//
// A lane keeps its candidate in every iteration of an event, so the candidate position's
// last-update time and the event's decay code are read once per event; iterations differ
// only in their channels, so each iteration's operands are read while the previous one
// computes.  Spikes: iteration-major, then lane = (channel, candidate) order, which is
// ascending neuron id oc*H*W + y*W + x, the order of salt_core/stream.py:24-46.
//
// Work decomposition.  A wave is one stream x one group of Gw channels.  With one group
// per stream (ncg = 1) the waves of a work-group are spw independent streams that share
// the tables, the weight codes and the decay table, with no barrier after the set-up;
// with several groups (small batches) the work-group is one stream whose waves exchange
// per-chunk spike counts behind one barrier per 64-event chunk, as conv_layer_kernel's do.
#pragma once

#include "conv_kernel.hpp"

namespace salt {

constexpr int kPackMaxNC = 5;       // classes NC*NC <= 25 (LDS tables)
constexpr int kPackMaxBlockWaves = 8;
constexpr int kPackRecBufs = 2;
constexpr int kPackEvtBufs = 3;
constexpr int kPackRecs = kWave + 3;  // a chunk's events + three empty records read ahead

struct PackArgs {
  ConvGeom g;
  int ncls;             // NC * NC
  int ncg, Gw, spw, B;  // channel groups per stream, channels per group, streams per WG
  int P;                // channel slots per wave (real + zero); slot P is the spare plane
  int VS, QS;           // words per register slot / code slot in LDS
  Quant qz;
  const int32_t* table;
  const void* q;
  int q_bits;
  int L;
  const float* times;
  const int32_t* src;
  const int32_t* n_real;
  int cap, fill_pads;
  float* out_t;
  int32_t* out_s;
  int32_t* out_n;
  int32_t* v_final;
  int32_t* v_min;
  int32_t* v_max;
  int32_t* stats;
};

// Iterations and channels per iteration of a class of n candidates for Gw channels.
__host__ __device__ inline void pack_class_split(int n, int Gw, int& I, int& G) {
  const int gmax = min(Gw, kWave / n);
  I = (Gw + gmax - 1) / gmax;
  G = (Gw + I - 1) / I;
}

// Channel slots a wave needs: every class's I * G (slots Gw.. are zero planes).
__host__ __device__ inline int pack_slots(int NC, int Gw, int* imax) {
  int P = Gw, im = 1;
  for (int h = 1; h <= NC; ++h)
    for (int w = 1; w <= NC; ++w) {
      int I, G;
      pack_class_split(h * w, Gw, I, G);
      P = max(P, I * G);
      im = max(im, I);
    }
  if (imax) *imax = im;
  return P;
}

// LDS layout of a packed work-group, in 4-byte words: shared part (decay table, class
// info, lane tables, spike map, weight codes of every channel group, reductions), one
// region per stream (records, event info, queue counts), one region per wave (spike
// ballots, per-position entries, registers, extremes, thresholds).
struct PackLds {
  int ext, cinfo, lt4, lsq, wmap, codes, red, shared_words;
  int rec, rec1, evt, nev, cnt, stream_words;
  int stg, wcnt, tc, v, mn, mx, th, wave_words;
  int streams, waves, words;
};

__host__ __device__ inline PackLds pack_lds_layout(int n_table, int ncls, int ncg, int spw,
                                                   int P, int VS, int QS, int PWs, int imax,
                                                   bool ext, bool vtha, bool notrunc) {
  PackLds l;
  int o = 0;
  l.ext = o;   o += n_table + 2;
  l.cinfo = o; o += 2 * ncls;
  o = (o + 3) & ~3;
  l.lt4 = o;   o += 4 * kWave * ncls;   // int4 {V, code, time-entry offsets, V stride}
  l.lsq = o;   o += kWave * ncls;       // code stride
  l.wmap = o;  o += 2 * kWave * ncls;   // int2 {channel slot, plane offset} per ballot bit
  l.codes = o; o += ncg * (P + 1) * QS;
  l.red = o;   o += 4 * kPackMaxBlockWaves;
  o = (o + 3) & ~3;
  l.shared_words = o;
  int s = 0;
  l.rec = s;   s += kPackRecBufs * kPackRecs * 4;  // int4 {t, position * 4, code * 4,
                                                   //       class | iterations << 8}
  l.rec1 = s;  s += kPackRecBufs * kPackRecs * 2;  // int2 {event index, 0}
  l.evt = s;   s += kPackEvtBufs * kWave * 4;      // int4 {t, plane position, class, 0}
  l.nev = s;   s += 4;
  l.cnt = s;   s += notrunc ? PWs : 0;
  s = (s + 3) & ~3;
  l.stream_words = s;
  int w = 0;
  l.stg = w;   w += 2 * kWave * imax * 2;          // uint64 ballot per (chunk event, iteration), x2
  l.wcnt = w;  w += 2 * kWave;
  l.tc = w;    w += (notrunc ? 1 : 2) * PWs;
  l.v = w;     w += (P + 1) * VS;
  l.mn = w;    w += ext ? (P + 1) * VS : 0;
  l.mx = w;    w += ext ? (P + 1) * VS : 0;
  l.th = w;    w += vtha ? (P + 1) * VS : 0;
  w = (w + 3) & ~3;
  l.wave_words = w;
  l.streams = l.shared_words;
  l.waves = l.streams + spw * l.stream_words;
  l.words = l.waves + spw * ncg * l.wave_words;
  return l;
}

// 16- and 8-byte LDS loads by byte address (through clang vector types, which load from
// address space 3 where HIP's int4/int2 do not).
typedef int salt_v4i __attribute__((ext_vector_type(4)));
typedef int salt_v2i __attribute__((ext_vector_type(2)));
__device__ __forceinline__ int4 lds_ld4(int addr) {
  const salt_v4i v = *reinterpret_cast<const __attribute__((address_space(3))) salt_v4i*>(
      (uintptr_t)(uint32_t)addr);
  return make_int4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ int2 lds_ld2(int addr) {
  const salt_v2i v = *reinterpret_cast<const __attribute__((address_space(3))) salt_v2i*>(
      (uintptr_t)(uint32_t)addr);
  return make_int2(v.x, v.y);
}

// Byte addresses (LDS) one wave's event loop uses.
struct PackWave {
  int rec, rec1;      // record buffers of the chunk
  int lt4, lsq;       // lane tables (already offset by this lane)
  int extb;           // decay table
  int vb, qb, tb;     // this wave's registers, codes, per-position entries
  int vspare, qzero;  // spare register (slot P), zero code (slot P)
  int dmn, dmx, dth;  // registers -> extremes / thresholds
  int mql;
  uint32_t nt1;       // n_table + 1
  uint64_t* stg;      // this chunk's ballots
  int32_t* wcnt;      // this chunk's spikes per event
};

// The events of one decoded chunk (salt_core/quant/scan.py:22-52 per update).  vt: the
// uniform threshold (none/scalar); VTHA: per-neuron thresholds beside the registers.
// NOTRUNC: every candidate event is a real queue column (max_queue_len >= stream length);
// otherwise a position whose queue is full drops the event (connectivity/conv.py:57-99).
//
// Software pipeline: event e+1's operands -- its decay code and
// every iteration's registers and codes -- are read right after event e's register
// writes (a wave's LDS operations complete in program order), so an event waits for one
// LDS round trip.  The
// records run three events ahead, the lane constants two and the per-position entries
// one (read after the previous event's entry writes), so none of those reads is waited
// for where it is issued.
template <int IMAX, bool SAT, bool EXT, bool VTHA, bool NOTRUNC>
__device__ __forceinline__ void pack_events(const Quant& qz, const PackWave& c, int vt_uniform,
                                            int n_ev, int base, int& vmin_l, int& vmax_l) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int it = 0; it < IMAX; ++it) c.stg[lane * IMAX + it] = ~0ull;
  c.wcnt[lane] = 0;
  if (n_ev == 0) return;
  uint32_t sg_lo[IMAX], sg_hi[IMAX];
#pragma unroll
  for (int it = 0; it < IMAX; ++it) { sg_lo[it] = ~0u; sg_hi[it] = ~0u; }
  const int fa = qz.fa, rc = qz.rc;
  constexpr int kTsc = NOTRUNC ? 0 : 1;  // record position bytes -> entry bytes (shift)
  auto tc_load = [&](int addr) -> int2 {
    return NOTRUNC ? make_int2(lds_ld<int32_t>(addr), 0) : lds_ld_tc(addr);
  };
  auto rec_at = [&](int e) { return lds_ld4(c.rec + e * 16); };
  auto rec1_at = [&](int e) { return lds_ld2(c.rec1 + e * 8); };
  auto lconst = [&](int cls, int4& lc, int& sq) {
    lc = lds_ld4(c.lt4 + cls * (kWave * 16));
    sq = lds_ld<int32_t>(c.lsq + cls * (kWave * 4));
  };
  // An event's operands: decay code and, for each of the IMAX iterations, its register
  // address and the values read there.  Iterations past the event's count work on the
  // spare slot with the zero code (U = 0: no spike, neutral extremes), so every event
  // runs the same straight-line code (measured: uniform tests around the iterations cost
  // more than the iterations they skip).
  struct Ops {
    int A;
    int va[IMAX];
    int v[IMAX], q[IMAX], th[IMAX], mn[IMAX], mx[IMAX];
  };
  auto read_ops = [&](Ops& o, const int4& r, const int4& lc, int lsq, const int2& st, int nit) {
    const bool act = NOTRUNC || st.y < c.mql;
    // decay code: dt = 0 identity, 1..n table, > n zero (an unsigned clamp)
    o.A = lds_ld<int32_t>(c.extb + (int)(min((uint32_t)(r.x - st.x), c.nt1) << 2));
    const int va0 = act ? c.vb + r.y + lc.x : c.vspare, sv = act ? lc.w : 0;
    const int qa0 = act ? c.qb + r.z + lc.y : c.qzero, sq = act ? lsq : 0;
#pragma unroll
    for (int it = 0; it < IMAX; ++it) {
      const bool on = it == 0 || it < nit;  // every processed event has an iteration
      const int va = on ? va0 + it * sv : c.vspare, qa = on ? qa0 + it * sq : c.qzero;
      o.va[it] = va;
      o.v[it] = lds_ld<int32_t>(va);
      o.q[it] = lds_ld<int32_t>(qa);
      if (VTHA) o.th[it] = lds_ld<int32_t>(va + c.dth);
      if (EXT) {
        o.mn[it] = lds_ld<int32_t>(va + c.dmn);
        o.mx[it] = lds_ld<int32_t>(va + c.dmx);
      }
    }
  };
  // pipeline: records of e .. e+3, lane constants of e .. e+2, entries of e .. e+1
  int4 r = rec_at(0), rn = rec_at(1), rn2 = rec_at(2);
  int4 lc, lcn;
  int lsq, lsqn;
  lconst(r.w & 255, lc, lsq);
  lconst(rn.w & 255, lcn, lsqn);
  int ta = c.tb + (r.y << kTsc) + lc.z;
  int2 st = tc_load(ta);
  // record word w: class | iterations << 8
  int nit = __builtin_amdgcn_readfirstlane(r.w >> 8);
  int nitn = __builtin_amdgcn_readfirstlane(rn.w >> 8);
  Ops o;
  read_ops(o, r, lc, lsq, st, nit);

  auto event = [&](int e) {
    // this event's positions: last-update time (and queue count), after their reads
    if (NOTRUNC)
      lds_st<int32_t>(ta, r.x);
    else
      lds_st_tc(ta, st.y < c.mql ? r.x : st.x, st.y + 1);
    // the next event's entries, after that write; records three ahead; lane constants two
    const int tan = c.tb + (rn.y << kTsc) + lcn.z;
    const int2 stn = tc_load(tan);
    const int4 rn3 = rec_at(e + 3);
    int4 lcn2;
    int lsqn2;
    lconst(rn2.w & 255, lcn2, lsqn2);
    const int nitn2 = __builtin_amdgcn_readfirstlane(rn2.w >> 8);
    asm volatile("" ::: "memory");
    // the iterations, their chains interleaved (written phase by phase: a dependent VALU
    // instruction waits for its operand, an independent one does not)
    int32_t u[IMAX], f[IMAX];
    uint64_t bal[IMAX];
#pragma unroll
    for (int it = 0; it < IMAX; ++it) u[it] = decay_mul_wide(o.v[it], o.A, fa, rc);
#pragma unroll
    for (int it = 0; it < IMAX; ++it) u[it] = (int32_t)((uint32_t)u[it] + (uint32_t)o.q[it]);
#pragma unroll
    for (int it = 0; it < IMAX; ++it) f[it] = fit_bits<SAT>(u[it], qz);
#pragma unroll
    for (int it = 0; it < IMAX; ++it) {
      const bool keep = f[it] < (VTHA ? o.th[it] : vt_uniform);
      bal[it] = __ballot(keep);  // the lanes that kept their value
      lds_st<int32_t>(o.va[it], keep ? f[it] : 0);
    }
#pragma unroll
    for (int it = 0; it < IMAX; ++it) {
      vmin_l = min(vmin_l, u[it]);
      vmax_l = max(vmax_l, u[it]);
      if (EXT) {
        lds_st<int32_t>(o.va[it] + c.dmn, min(o.mn[it], u[it]));
        lds_st<int32_t>(o.va[it] + c.dmx, max(o.mx[it], u[it]));
      }
    }
    asm volatile("" ::: "memory");  // the next event's reads come after these writes
    read_ops(o, rn, lcn, lsqn, stn, nitn);
    // ballots staged into lane e after the next event's reads have gone out (the lane
    // index passes through an empty asm so that the writes stay here)
    int el = e;
    asm volatile("" : "+s"(el));
#pragma unroll
    for (int it = 0; it < IMAX; ++it) stage_to_lane(sg_lo[it], sg_hi[it], bal[it], el);
    r = rn; lc = lcn; lsq = lsqn; st = stn; ta = tan; nit = nitn;
    rn = rn2; lcn = lcn2; lsqn = lsqn2; nitn = nitn2;
    rn2 = rn3;
  };
  // two events per loop iteration: the carried state needs no register copies
  int e = 0;
  for (; e + 1 < n_ev; e += 2) {
    event(e);
    event(e + 1);
  }
  if (e < n_ev) event(e);
  if (lane < n_ev) {
    const int jc = rec1_at(lane).x - base;  // the event's index within the chunk
    int nsp = 0;
#pragma unroll
    for (int it = 0; it < IMAX; ++it) {
      const uint64_t kept = ((uint64_t)sg_hi[it] << 32) | sg_lo[it];
      c.stg[jc * IMAX + it] = kept;
      nsp += __popcll(~kept);
    }
    c.wcnt[jc] = nsp;
  }
}

template <int IMAX, bool SAT, bool EXT, bool VTHA, bool NOTRUNC>
__global__ void __launch_bounds__(kWave * kPackMaxBlockWaves) __attribute__((amdgpu_waves_per_eu(1, 2)))
conv_packed_kernel(PackArgs a) {
  extern __shared__ int32_t smem[];
  const ConvGeom& g = a.g;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int nthr = blockDim.x;
  const int ks = wv / a.ncg, cg = wv - ks * a.ncg;  // stream slot, channel group
  const int b = blockIdx.x * a.spw + ks;
  const bool live = b < a.B;
  const int Gw = a.Gw, P = a.P, VS = a.VS, QS = a.QS, NC = g.NC;
  const int oc0 = cg * Gw;
  const int ocn = max(0, min(Gw, g.OC - oc0));
  const int H = g.H, W = g.W, Wp = g.Wp, PWs = H * Wp;
  const int ICKK = g.IC * g.K * g.K;
  const Quant& qz = a.qz;
  const PackLds lay = pack_lds_layout(qz.n_table, a.ncls, a.ncg, a.spw, P, VS, QS, PWs, IMAX,
                                      EXT, VTHA, NOTRUNC);
  constexpr int kTcb = NOTRUNC ? 4 : 8;  // bytes per per-position entry
  int32_t* const sreg = smem + lay.streams + ks * lay.stream_words;
  int32_t* const wreg = smem + lay.waves + wv * lay.wave_words;
  const int32_t* const swave0 = smem + lay.waves + ks * a.ncg * lay.wave_words;
  int32_t* const ext = smem + lay.ext;
  int2* const cinfo = reinterpret_cast<int2*>(smem + lay.cinfo);
  int4* const lt4 = reinterpret_cast<int4*>(smem + lay.lt4);
  int32_t* const lsq = smem + lay.lsq;
  int2* const wmap = reinterpret_cast<int2*>(smem + lay.wmap);
  int32_t* const red = smem + lay.red;
  int4* const recs = reinterpret_cast<int4*>(sreg + lay.rec);
  int2* const recs1 = reinterpret_cast<int2*>(sreg + lay.rec1);
  int4* const evt = reinterpret_cast<int4*>(sreg + lay.evt);
  int32_t* const nev = sreg + lay.nev;
  int32_t* const cnt = sreg + lay.cnt;
  uint64_t* const stgs = reinterpret_cast<uint64_t*>(wreg + lay.stg);
  int32_t* const Vs = wreg + lay.v;

  // ---- shared: decay table, class tables, codes
  load_ext_table(ext, a.table, qz.n_table, qz.fa, tid, nthr);
  for (int i = tid; i < a.ncls * kWave; i += nthr) {
    const int cls = i / kWave, l = i - cls * kWave;
    const int h = cls / NC + 1, w = cls - (cls / NC) * NC + 1, n = h * w;
    int I, G;
    pack_class_split(n, Gw, I, G);
    if (l < G * n) {
      const int slot = l / n, cand = l - slot * n, dy = cand / w, dx = cand - dy * w;
      lt4[i] = make_int4((slot * VS + dy * Wp + dx) * 4, (slot * QS - dy * g.S * g.K - dx * g.S) * 4,
                         (dy * Wp + dx) * kTcb, G * VS * 4);
      lsq[i] = G * QS * 4;
      wmap[i] = make_int2(slot, dy * W + dx);
    } else {  // past the class's lanes: the spare slot, no stride
      lt4[i] = make_int4(P * VS * 4, P * QS * 4, 0, 0);
      lsq[i] = 0;
      wmap[i] = make_int2(-1, 0);
    }
    if (l == 0) cinfo[cls] = make_int2(I, G);
  }
  for (int i = tid; i < a.ncg * (P + 1) * QS; i += nthr) {
    const int gi = i / ((P + 1) * QS), rem = i - gi * ((P + 1) * QS);
    const int s = rem / QS, k = rem - s * QS;
    const int oc = gi * Gw + s;
    // codes pre-shifted, q * 2^f_V in two's complement (U = D + q*2^f_V); zero slots
    smem[lay.codes + i] = (s < Gw && oc < g.OC && k < ICKK)
                              ? (int32_t)((uint32_t)load_code_bits(a.q, (size_t)oc * ICKK + k, a.q_bits)
                                          << qz.fV)
                              : 0;
  }
  // ---- this wave's state
  const int vwords = (P + 1) * VS;
  for (int i = lane; i < vwords; i += kWave) {
    Vs[i] = 0;
    if (EXT) { wreg[lay.mn + i] = 0; wreg[lay.mx + i] = 0; }
    if (VTHA) {
      const int s = i / VS, p = i - s * VS, row = p / Wp, col = p - row * Wp;
      int t = INT_MAX;
      if (s < ocn && row < H && col < W) {
        const int oc = oc0 + s;
        t = qz.vth_kind == SALT_VTH_PER_NEURON ? qz.vth[(size_t)oc * g.HW + row * W + col]
                                                : qz.vth[oc];
      }
      wreg[lay.th + i] = t;
    }
  }
  for (int i = lane; i < (NOTRUNC ? 1 : 2) * PWs; i += kWave) wreg[lay.tc + i] = 0;
  const bool dec = cg == 0;  // the stream's first wave decodes its events
  if (dec) {
    if (NOTRUNC)
      for (int i = lane; i < PWs; i += kWave) cnt[i] = 0;
    if (lane < kPackRecs - kWave)  // the records after a full chunk: nothing
      for (int bf = 0; bf < kPackRecBufs; ++bf) {
        recs[bf * kPackRecs + kWave + lane] = make_int4(0, 0, 0, 0);
        recs1[bf * kPackRecs + kWave + lane] = make_int2(-1, 0);
      }
  }
  __syncthreads();
  // With one wave per stream the waves never meet again; slots past the batch leave.
  // With several channel groups the work-group's waves meet once per chunk, so every wave
  // runs to the work-group's longest stream (a slot past the batch has no events).
  if (!live && a.ncg == 1) return;

  const int b0 = lds_addr(smem);
  PackWave c;
  c.lt4 = b0 + (lay.lt4 + lane * 4) * 4;
  c.lsq = b0 + (lay.lsq + lane) * 4;
  c.extb = b0 + lay.ext * 4;
  c.vb = (int)lds_addr(Vs);
  c.qb = b0 + (lay.codes + cg * (P + 1) * QS) * 4;
  c.tb = (int)lds_addr(wreg + lay.tc);
  c.vspare = c.vb + P * VS * 4;
  c.qzero = c.qb + P * QS * 4;
  c.dmn = (lay.mn - lay.v) * 4;
  c.dmx = (lay.mx - lay.v) * 4;
  c.dth = (lay.th - lay.v) * 4;
  c.mql = g.mql;
  c.nt1 = (uint32_t)qz.n_table + 1u;
  const int vt_uniform = qz.vth_kind == SALT_VTH_SCALAR ? qz.vth_scalar : INT_MAX;

  const int L = a.L;
  auto real_count = [&](int bi) {
    const int nr = bi < a.B ? a.n_real[bi] : 0;
    return nr < 0 ? 0 : (nr < L ? nr : L);
  };
  const int n_eff = real_count(b);
  int n_grp = n_eff;
  if (a.ncg > 1) {
    n_grp = 0;
    for (int i = lane; i < a.spw; i += kWave) n_grp = max(n_grp, real_count(blockIdx.x * a.spw + i));
    n_grp = __builtin_amdgcn_readfirstlane(wave_max(n_grp));
  }
  const int nchunks = (n_grp + kWave - 1) / kWave;
  const float* tbp = a.times + (size_t)(live ? b : 0) * L;
  const int32_t* sbp = a.src + (size_t)(live ? b : 0) * L;
  int vmin_l = 0, vmax_l = 0;
  int out_base = 0;
  const int jl = n_eff - 1;
  float t_n = 0.0f;
  int s_n = -1;
  if (dec && jl >= 0) {
    t_n = tbp[min(lane, jl)];
    s_n = sbp[min(lane, jl)];
  }
  const int n_src = g.IC * g.HWin;
  // Decoding wave: chunk k into record buffer k % 2, event info into buffer k % 3.
  auto decode = [&](int k) {
    const int bf = k & 1;
    const int j = k * kWave + lane;
    const int tv = time_ms(t_n), sv = s_n;
    if (jl >= 0) {
      const int j2 = min(j + kWave, jl);
      t_n = tbp[j2];
      s_n = sbp[j2];
    }
    const bool real = j < n_eff && sv >= 0;
    // source -> (channel, row, column); a source past the input is clamped into it
    // (memory safety only: the host rejects such ids)
    const int s = real ? min(sv, n_src - 1) : 0;
    int ch, y, x, oy0, ox0, yhi, xhi;
    if (n_src <= (1 << 22)) {
      ch = div_small(s, g.HWin, g.rHWin);
      const int rem = s - ch * g.HWin;
      y = div_small(rem, g.Win, g.rWin);
      x = rem - y * g.Win;
      oy0 = div_small(y + g.P - g.K + g.S + g.K * g.S, g.S, g.rS) - g.K;
      ox0 = div_small(x + g.P - g.K + g.S + g.K * g.S, g.S, g.rS) - g.K;
      yhi = div_small(y + g.P, g.S, g.rS);
      xhi = div_small(x + g.P, g.S, g.rS);
    } else {
      ch = s / g.HWin;
      const int rem = s - ch * g.HWin;
      y = rem / g.Win;
      x = rem - y * g.Win;
      oy0 = floordiv_pos(y + g.P - g.K + g.S, g.S);
      ox0 = floordiv_pos(x + g.P - g.K + g.S, g.S);
      yhi = (y + g.P) / g.S;
      xhi = (x + g.P) / g.S;
    }
    // the candidate rectangle within the plane (connectivity/conv.py:15-29)
    const int oyb = max(oy0, 0), oxb = max(ox0, 0);
    const int h = min(yhi, H - 1) - oyb + 1, w = min(xhi, W - 1) - oxb + 1;
    const bool rel = real && h > 0 && w > 0;
    const int cls = rel ? (h - 1) * NC + (w - 1) : 0;
    const int p0 = oyb * Wp + oxb;
    const int q0 = ch * g.K * g.K + (y + g.P - oyb * g.S) * g.K + (x + g.P - oxb * g.S);
    if (NOTRUNC && rel)
      for (int dy = 0; dy < h; ++dy)
        for (int dx = 0; dx < w; ++dx) atomicAdd(&cnt[p0 + dy * Wp + dx], 1);
    const int nit = rel ? cinfo[cls].x : 0;
    const uint64_t relm = __ballot(rel);
    const int n = __popcll(relm);
    const int slot = rel ? lanes_below(relm) : n + lanes_below(~relm);
    recs[bf * kPackRecs + slot] =
        rel ? make_int4(tv, p0 * 4, q0 * 4, cls | (nit << 8)) : make_int4(0, 0, 0, 0);
    recs1[bf * kPackRecs + slot] = make_int2(j, nit);
    evt[(k % kPackEvtBufs) * kWave + lane] = make_int4(tv, oyb * W + oxb, cls, 0);
    if (lane == 0) nev[bf] = n;
  };
  // Every wave: its own spikes of chunk k at their places in the stream's output, ordered
  // (event, channel group, iteration, bit) = (event, ascending neuron id).  Lane = the
  // event's index in the chunk.
  auto walk = [&](int k) {
    const int bf = k & 1;
    int tot = 0, before = 0;
    for (int g2 = 0; g2 < a.ncg; ++g2) {
      const int cw = swave0[g2 * lay.wave_words + lay.wcnt + bf * kWave + lane];
      tot += cw;
      before += g2 < cg ? cw : 0;
    }
    if (__ballot(tot != 0) == 0) return;  // no spike in the chunk
    const int incl = wave_incl_scan(tot);
    const int total = __builtin_amdgcn_readlane(incl, kWave - 1);
    const int4 ev = evt[(k % kPackEvtBufs) * kWave + lane];
    const float te = ms_time(ev.x);
    const int G = cinfo[ev.z].y;
    int pos = out_base + (incl - tot) + before;
    const uint64_t* const st = stgs + bf * kWave * IMAX + lane * IMAX;
#pragma unroll
    for (int it = 0; it < IMAX; ++it) {
      uint64_t bits = ~st[it];
      while (bits) {
        const int kb = __builtin_ctzll(bits);
        bits &= bits - 1;
        const int2 m = wmap[ev.z * kWave + kb];
        const int oc = oc0 + it * G + m.x;
        if (pos < a.cap) {
          a.out_t[(size_t)b * a.cap + pos] = te;
          a.out_s[(size_t)b * a.cap + pos] = oc * g.HW + ev.y + m.y;
        }
        ++pos;
      }
    }
    out_base += total;
  };

  if (dec && nchunks > 0) decode(0);
  if (a.ncg > 1) __syncthreads();
  for (int k = 0; k < nchunks; ++k) {
    const int bf = k & 1;
    if (dec && k + 1 < nchunks) decode(k + 1);
    if (k > 0) walk(k - 1);
    c.rec = (int)lds_addr(reinterpret_cast<int32_t*>(recs + bf * kPackRecs));
    c.rec1 = (int)lds_addr(reinterpret_cast<int32_t*>(recs1 + bf * kPackRecs));
    c.stg = stgs + bf * kWave * IMAX;
    c.wcnt = wreg + lay.wcnt + bf * kWave;
    const int n_ev = __builtin_amdgcn_readfirstlane(nev[bf]);
    pack_events<IMAX, SAT, EXT, VTHA, NOTRUNC>(qz, c, vt_uniform, n_ev, k * kWave, vmin_l, vmax_l);
    if (a.ncg > 1) __syncthreads();
  }
  if (nchunks > 0) walk(nchunks - 1);

  // catch-up column and final registers (conv_finish reads the channel slots 0..ocn-1)
  if (!live) {  // a slot past the batch: meet the stream's last barrier, write nothing
    if (a.ncg > 1) __syncthreads();
    return;
  }
  ConvLane fin;
  fin.Vs = Vs;
  fin.mn = wreg + lay.mn;
  fin.mx = wreg + lay.mx;
  fin.tc = reinterpret_cast<int2*>(wreg + lay.tc);
  fin.cnt = cnt;
  fin.ext = ext;
  fin.mql = g.mql;
  fin.ntab = qz.n_table;
  const int T = n_eff > 0 ? time_ms(tbp[n_eff - 1]) : 0;
  int maxcnt = conv_finish<EXT, NOTRUNC>(qz, fin, lane, T, ocn, H * W, W, Wp, VS,
                                         (size_t)b * (g.OC * g.HW) + (size_t)oc0 * g.HW, g.HW,
                                         a.v_final, a.v_min, a.v_max, vmin_l, vmax_l);
  vmin_l = wave_min(vmin_l);
  vmax_l = wave_max(vmax_l);
  if (a.ncg > 1) {  // the stream's extremes over its waves
    if (lane == 0) {
      red[wv * 4 + 0] = vmin_l;
      red[wv * 4 + 1] = vmax_l;
      red[wv * 4 + 2] = maxcnt;
    }
    __syncthreads();
    if (cg != 0) return;
    for (int w2 = wv + 1; w2 < wv + a.ncg; ++w2) {
      vmin_l = min(vmin_l, red[w2 * 4 + 0]);
      vmax_l = max(vmax_l, red[w2 * 4 + 1]);
      maxcnt = max(maxcnt, red[w2 * 4 + 2]);
    }
  }
  const int ovf = (vmin_l < -qz.half || vmax_l > qz.half - 1) ? 1 : 0;
  if (lane == 0) {
    a.out_n[b] = out_base;
    a.stats[b * 4 + 0] = vmin_l;
    a.stats[b * 4 + 1] = vmax_l;
    a.stats[b * 4 + 2] = maxcnt + 1;
    a.stats[b * 4 + 3] = ovf;
  }
  if (a.fill_pads)
    for (int i = min(out_base, a.cap) + lane; i < a.cap; i += kWave) {
      a.out_t[(size_t)b * a.cap + i] = kPadTime;
      a.out_s[(size_t)b * a.cap + i] = 0;
    }
}

}  // namespace salt
