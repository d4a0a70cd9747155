// Event-driven integer conv layer (salt_core/layers/conv.py:124-149 with the queue of
// salt_core/connectivity/conv.py and the scan of salt_core/quant/scan.py:22-132).
//
// A work-group owns one stream and a band of R output rows (in-kernel output: the whole
// plane).  Its channel-group waves split that band into ncg channel groups x nsb
// sub-bands of Rw rows; each processes, in order, the stream's events whose candidate
// rows meet its sub-band, as decoded by the sub-band's helper wave, which with few
// channel groups also places the sub-band's spikes in the output (so a channel group's
// wave runs nothing but its events: the decode and the placement take a quarter of a
// stream's time when the channel groups do them themselves, measured on one stream);
// with many, each channel-group wave places its own.  Everything a wave touches
// per event lives in LDS: registers V[channel slot][position], per-position (last-update
// time, queue count), and -- shared -- the weight codes of its channel group and the
// extended decay table.
//
// Lane mapping.  NC = (k-1)//s + 1 candidate rows (and columns) per input event and
// NC2 = NC*NC candidates; lane l is channel slot l / NC2 (+ Gi per iteration) and
// candidate (dy, dx) = divmod(l % NC2, NC).  Relative to an event's first candidate
// (oy0, ox0) = (ceil((y+P-K+1)/S), ceil((x+P-K+1)/S)) every address a lane needs is an
// event-uniform base plus a lane constant:
//   V slot    = ((oy0-r0)*Wp + ox0) + [slot*VS + dy*Wp + dx]
//   weight    = (c*K*K + (y+P-oy0*S)*K + (x+P-ox0*S)) + [slot*QS - dy*S*K - dx*S]
// where Wp >= W is the row stride of the position arrays in LDS and VS, QS the slot
// strides, chosen on the host so that a wave's accesses spread over the LDS banks
// (the padding columns are never touched).  The helper wave turns 64 events at a time
// (one per lane) into LDS records: those two bases, the time and a 64-bit mask of the
// candidates in the output plane and its sub-band; the loop reads one record per event
// (a broadcast).
//
// No lane predicates in the event loop.  A lane without an update this event (no
// candidate, or a full queue) reads and writes spare words (registers zero, thresholds
// unreachable) and a zero code: a zero register and a zero
// code give U = 0 and never fire, and the extremes start at 0.  Channel slots past a
// wave's channels likewise hold zero codes and an unreachable threshold.
//
// Output.  With the whole plane in the work-group, each channel-group wave stores the
// ballot of its spikes per (chunk event, iteration) and its spike count per chunk event
// in LDS; in the next chunk the helper wave places every group's spikes in the stream's
// output (or each wave its own), in the order (event, channel group, iteration, lane) =
// (event, ascending neuron id) of salt_core/stream.py:24-46, from a scan of all the
// stream's waves' counts.  With
// several work-groups per stream (state above the LDS size: bands of rows) the waves
// stage the same ballots; in the next chunk, for each event with a spike in the band, the
// helper stores every group's ballots as 64-bit spike words in global memory, in the
// event's slot for this band, and marks the slot valid; a compaction kernel orders them.
// Nothing is stored for an event without a spike in the band, and only the validity
// words need clearing before the launch.
//
// One barrier per 64-event chunk, none inside the event loop: a wave's LDS operations
// complete in program order, so event e+1 reads what event e wrote.  The helper decodes
// the next chunk (and places or stores the previous one's spikes) while the channel
// groups run this one (double-buffered records and ballots).
#pragma once

#include "salt_device.hpp"

namespace salt {

constexpr int kConvMaxWaves = 8;     // channel-group waves per stream (groups x sub-bands)
constexpr int kConvBlockWaves = 16;  // waves per work-group (streams x waves per stream)

// Waves of a work-group: per stream, its channel-group waves and one helper per sub-band.
__host__ __device__ inline int conv_block_waves(int spw, int ncg, int nsb) {
  return spw * (ncg * nsb + nsb);
}

// Geometry of a conv layer as the device code uses it.
struct ConvGeom {
  int IC, Win, HWin, OC, K, S, P, H, W, HW, NC, NC2, mql;
  int Wp;  // row stride of the per-position arrays in LDS (>= W)
  float rHWin, rWin, rS;  // 1/HWin, 1/Win, 1/S (for div_small)
};

struct ConvArgs {
  ConvGeom g;
  // partition: G channels per channel group in NIT iterations of Gi slots; ncg channel
  // groups x nsb sub-bands of Rw rows per work-group; R rows per work-group
  int G, Gi, ncg, nsb, Rw, R;
  // spw streams per work-group (whole-plane plans), B streams in all
  int spw, B;
  // Row-band plans: the events whose candidate rows meet each (stream, band), as original
  // indices in order -- band (b, x) has bcnt[b * gridDim.x + x] of them from
  // blist + b * bcap + boff[b * gridDim.x + x].  Null: every work-group reads its stream.
  const int32_t* blist;
  const int32_t* bcnt;
  const int32_t* boff;
  int bcap;
  int VS, QS;  // slot strides of the registers and the weight codes in LDS
  // quantisation
  Quant qz;
  const int32_t* table;
  const void* q;
  int q_bits;
  // events
  int L;
  const float* times;
  const int32_t* src;
  const int32_t* n_real;
  // outputs
  int cap, fill_pads, merge;  // merge: one work-group per stream, ordered output in-kernel
  // merge mode: 1 = the helper waves place every channel group's spikes, 0 = each
  // channel-group wave places its own (the helper only decodes)
  int hwalk;
  // 1: the helper waves run at issue priority 1 (their per-chunk work is heavy), 0: at 0
  int hprio;
  float* out_t;
  int32_t* out_s;
  int32_t* out_n;
  int32_t* v_final;
  int32_t* v_min;
  int32_t* v_max;
  int32_t* stats;
  // Row-band plans: an event reaches at most nslots consecutive bands, band x filling slot
  // x % nslots of the event.  words: [B][L][nslots][ncg][NIT] spike words (lane l of
  // channel group g's iteration it = slot l / NC2, candidate l % NC2), stored only for
  // events with a spike in the band; valid: [B][L] bit per slot stored.
  uint64_t* words;
  uint32_t* valid;
  int nslots;
  int32_t* seg_cnt;  // row bands: spikes per (stream, kCompactSeg events), [B][nseg]
  int nseg;
};

// Spare positions.  A lane without a candidate in an event reads and writes a spare
// position of its own, which no event touches; every lane's address is then one base
// (the event's position base, or the lane's spare base) plus its lane constant.  Bands
// of at least NC rows (pad) keep the spares in padding columns: position (dy, W + dx) for
// candidate offset (dy, dx), with rows of Wp >= W + NC; smaller bands keep NC2 spare
// words after their PWs positions.
__host__ __device__ inline bool conv_spare_pad(int Rw, int NC) { return Rw >= NC; }
// Words of a per-position array (registers of a slot, (time, count) entries).
__host__ __device__ inline int conv_pos_words(int PWs, int NC2, bool pad) {
  return pad ? PWs : PWs + NC2;
}

// LDS layout of a conv_layer_kernel work-group, in 4-byte words: a shared part (decay
// table, ballot-bit map, reduction slots, int32 weight codes per channel group), one
// region per (stream, sub-band) -- the decoded records and what the decode keeps -- then
// one region per wave (spw streams x ncg x nsb waves).
struct ConvLds {
  int ext, lanemap, red, qs, shared_words;                      // shared
  int rec, rec1, evt, nev, cnt, band_words;                     // per (stream, sub-band)
  int stg, wcnt, tc, vthc, v, mn, mx, th, wave_words;           // per wave
  int waves;  // word offset of the first wave region
  int vs, qst, tcn;
  int words;
};

// Record buffers (chunks in flight between the decode and the event loop) and event-info
// buffers (chunks in flight between the decode and the output walk).
constexpr int kConvRecBufs = 2;
constexpr int kConvEvtBufs = 3;
// Records per buffer: a chunk's steps and two steps that cover nothing, one record per
// step, or two (pair: the events of the step's two half-waves).
__host__ __device__ inline int conv_recs(bool pair) { return (pair ? 2 : 1) * (kWave + 2); }

// PWs: padded positions of a band (rows x Wp); npos = conv_pos_words(); vs >= npos and
// qs >= ICKK + 1: slot strides (a slot's codes are followed by a zero).
// tsplit (no queue truncation possible): the per-position entries are last-update times
// alone, and the queue counts a separate array (kept by the decode, read at the end).
// pair: two events per step (one per half-wave).
__host__ __device__ inline ConvLds conv_lds_layout(int n_table, int spw, int ncg, int nsb,
                                                   int Gp, int nit, int vs, int qs, int PWs,
                                                   int npos, bool ext, bool vthn, bool tsplit,
                                                   bool pair) {
  ConvLds l;
  l.vs = vs;
  l.qst = qs;
  l.tcn = npos;
  int o = 0;
  l.ext = o;     o += n_table + 2;
  l.lanemap = o; o += 2 * kWave;  // int2 {slot, position offset} per ballot bit
  l.red = o;     o += 4 * kConvBlockWaves;
  l.qs = o;      o += ncg * Gp * l.qst;
  o = (o + 3) & ~3;
  l.shared_words = o;
  int bw = 0;
  // Two steps more than a chunk's events: the loop reads two steps ahead.
  const int nrec = kConvRecBufs * conv_recs(pair);
  l.rec = bw;  bw += nrec * 4;                      // int4 {t, V base, weight base, mask low}
  l.rec1 = bw; bw += nrec * 2;                      // int2 {mask high, event index}
  l.evt = bw;  bw += kConvEvtBufs * kWave * 2;      // int2 {t, plane position} per chunk event
  l.nev = bw;  bw += 4;                             // steps of the chunk, per record buffer
  l.cnt = bw;  bw += tsplit ? PWs : 0;              // queue counts (tsplit)
  bw = (bw + 3) & ~3;
  l.band_words = bw;
  l.waves = l.shared_words + spw * nsb * bw;
  int w = 0;
  l.stg = w;  w += 2 * kWave * nit * 2;  // uint64 spike ballot per (chunk event, iteration), x2
  l.wcnt = w; w += 2 * kWave;            // spikes per chunk event, x2
  l.tc = w;   w += (tsplit ? 1 : 2) * l.tcn;  // {last-update time, queue count} or time
  l.vthc = w; w += Gp;
  l.v = w;    w += Gp * l.vs;
  l.mn = w;   w += ext ? Gp * l.vs : 0;
  l.mx = w;   w += ext ? Gp * l.vs : 0;
  l.th = w;   w += vthn ? Gp * l.vs : 0;
  w = (w + 3) & ~3;
  l.wave_words = w;
  l.words = l.waves + spw * ncg * nsb * w;
  return l;
}

// Per-lane constants and LDS pointers of one wave (see the file comment).  The event
// loop addresses LDS by byte offsets from the start of the work-group's LDS (where the
// decay table sits): records hold an event's position and code bases pre-scaled to
// bytes, and the lane constants below fold in this wave's region, so an address is one
// add (or shift-add) and a select.
struct ConvLane {
  int4* rec;
  int2* rec1;
  uint64_t* stg;         // this chunk's spike ballots
  int32_t* wcnt;         // this chunk's spikes per event
  int2* tc;
  const int32_t* ext;
  const int32_t* qs;     // weight codes q*2^f_V
  int32_t* Vs;
  int32_t* mn;
  int32_t* mx;
  int32_t* th;
  int32_t* cnt;         // tsplit: queue counts of the band's positions
  uint64_t lm;          // this lane's candidate bit (0 for lanes without a slot)
  int rh;               // pair: the lane's record of a step (its half-wave), else 0
  int lp, lv, lq;       // position / register / code offsets relative to an event's bases
  int q_zero;           // this lane's zero code
  int GiVS, GiQS;
  int cand, oc_lane, mql, ntab;
  // byte offsets from the LDS base, for the event loop
  int extb;                     // decay table
  int lvb, lqb, ltb;            // register, code, (time, count) entry of an event's base
  int q_zero_b;
  int sb;                       // spare base (records' units: position x 4)
  int GiVSb, GiQSb;             // per iteration
  int dmn, dmx, dth;            // register array -> extremes / per-neuron thresholds
};

// The LDS address of a pointer into the work-group's LDS.
__device__ __forceinline__ uint32_t lds_addr(const int32_t* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) int32_t*)p;
}

// Lane constants for a wave of Gi slots per iteration over a band of PWs positions
// (slot strides VS / QS), whose first channel is oc0; tcb: bytes per (time, count)
// entry (8, or 4 for times alone).  base: the work-group's LDS.  pair: each half-wave
// holds the same Gi slots for its own event.
__device__ __forceinline__ void conv_lane_setup(ConvLane& c, const ConvGeom& g, int lane,
                                                int Gi, int VS, int QS, int PWs, int oc0,
                                                int ntab, int tcb, const int32_t* base,
                                                bool pair) {
  const int ll = pair ? (lane & 31) : lane;  // the lane among its event's lanes
  const int slot0 = ll / g.NC2;
  c.cand = ll - slot0 * g.NC2;
  c.rh = pair ? lane >> 5 : 0;
  const int dy = c.cand / g.NC, dx = c.cand - (c.cand / g.NC) * g.NC;
  const bool lane_on = slot0 < Gi;
  const int slot_t = lane_on ? slot0 : 0;
  c.lm = lane_on ? (1ull << c.cand) : 0ull;
  c.lp = dy * g.Wp + dx;
  // Lanes without a slot are never covered and use slot 0's spare words (VS >=
  // conv_pos_words() keeps them inside slot 0's region).
  c.lv = slot_t * VS + c.lp;
  c.lq = slot_t * QS - dy * g.S * g.K - dx * g.S;
  c.q_zero = slot_t * QS + g.IC * g.K * g.K;
  c.GiVS = Gi * VS;
  c.GiQS = Gi * QS;
  c.oc_lane = oc0 + slot0;
  c.mql = g.mql;
  c.ntab = ntab;
  const int vw = (int)(c.Vs - base), qw = (int)(c.qs - base);
  const int tw = (int)(reinterpret_cast<const int32_t*>(c.tc) - base);
  const int b0 = (int)lds_addr(base);
  c.lvb = b0 + (vw + c.lv) * 4;
  c.lqb = b0 + (qw + c.lq) * 4;
  c.ltb = b0 + tw * 4 + c.lp * tcb;
  c.q_zero_b = b0 + (qw + c.q_zero) * 4;
  // spare position: (dy, W + dx) in the padding columns, or word PWs + cand
  const int spare = conv_spare_pad(PWs / g.Wp, g.NC) ? g.W + c.lp : PWs + c.cand;
  c.sb = (spare - c.lp) * 4;
  c.extb = (int)lds_addr(c.ext);
  c.GiVSb = c.GiVS * 4;
  c.GiQSb = c.GiQS * 4;
  c.dmn = (int)(c.mn - c.Vs) * 4;
  c.dmx = (int)(c.mx - c.Vs) * 4;
  c.dth = (int)(c.th - c.Vs) * 4;
}

// LDS access by byte address (the base is folded into the lane constants once, so the
// event loop adds nothing to an address).
template <typename T>
__device__ __forceinline__ T lds_ld(int addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) T*>((uintptr_t)(uint32_t)addr);
}
template <typename T>
__device__ __forceinline__ void lds_st(int addr, T v) {
  *reinterpret_cast<__attribute__((address_space(3))) T*>((uintptr_t)(uint32_t)addr) = v;
}
// (time, count) entries as one 64-bit word.
__device__ __forceinline__ int2 lds_ld_tc(int addr) {
  const uint64_t w = lds_ld<uint64_t>(addr);
  return make_int2((int)(uint32_t)w, (int)(uint32_t)(w >> 32));
}
__device__ __forceinline__ void lds_st_tc(int addr, int t, int cnt) {
  lds_st<uint64_t>(addr, ((uint64_t)(uint32_t)cnt << 32) | (uint32_t)t);
}

// Decodes the events of one chunk (connectivity/conv.py:15-43), one per lane (time tv,
// source sv, index j; real when j < n_eff and sv >= 0), against the rows [r0, r0+rn):
// records {time, position base * 4, code base * 4, candidate mask low} + {mask high,
// idx} for the events with a candidate there, compacted in order, followed by
// records with no candidate (mask 0) for the other lanes; with the two permanent ones
// at indices kWave and kWave + 1, the two records after a chunk's last event cover
// nothing, so the event loop reads two records ahead without a bounds test.  Returns
// the number of events with a candidate; oy0/ox0 = the event's first candidate row and
// column.
// cnt (queue counts of a wave that keeps them, else null): each event adds one to the
// count of every candidate position it has.
// PAIR: the records go to steps of two events instead, and the number of steps is
// returned (see below).  idx: the event's place in the decoded sequence (its stream index,
// or its place in a band's event list), the base of the chunk plus the lane.
template <bool PAIR>
__device__ __forceinline__ int conv_decode(const ConvGeom& g, const ConvLane& c, int tv,
                                           int sv, int j, int idx, int n_eff, int r0, int rn,
                                           int& oy0, int& ox0, int32_t* cnt) {
  const bool real = j < n_eff && sv >= 0;
  // source -> (channel, row, column); a source past the input is clamped into it (memory
  // safety only: the host rejects such ids)
  const int n_src = g.IC * g.HWin;
  const int s = real ? min(sv, n_src - 1) : 0;
  // Candidate output rows [ceil((y+P-K+1)/S), floor((y+P)/S)] within [r0, r0+rn) and
  // columns within [0, W) (connectivity/conv.py:15-29); ceil((a+1)/S) = floor((a+S)/S),
  // taken as floor((a+S+K*S)/S) - K to divide a non-negative number.
  int ch, y, x, yhi, xhi;
  if (n_src <= (1 << 22)) {  // every operand below 2^22: div_small
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
  const int dyA = max(oy0, r0) - oy0, dyB = min(yhi, r0 + rn - 1) - oy0;
  const int dxA = max(ox0, 0) - ox0, dxB = min(xhi, g.W - 1) - ox0;
  const bool rel = real && dyA <= dyB && dxA <= dxB;
  uint64_t m = 0;
  if (rel) {
    const uint64_t cols = (2ull << dxB) - (1ull << dxA);
    for (int d = dyA; d <= dyB; ++d) m |= cols << (d * g.NC);
  }
  const int p0 = (oy0 - r0) * g.Wp + ox0;
  const int q0 = ch * g.K * g.K + (y + g.P - oy0 * g.S) * g.K + (x + g.P - ox0 * g.S);
  if (cnt && rel)
    for (int d = dyA; d <= dyB; ++d)
      for (int dx = dxA; dx <= dxB; ++dx) atomicAdd(&cnt[p0 + d * g.Wp + dx], 1);
  const uint64_t relm = __ballot(rel);
  const int n = __popcll(relm);
  const int slot = rel ? lanes_below(relm) : n + lanes_below(~relm);
  if (!PAIR) {
    c.rec[slot] = make_int4(tv, p0 * 4, q0 * 4, (int)(uint32_t)m);
    c.rec1[slot] = make_int2((int)(uint32_t)(m >> 32), idx);
    return n;
  }
  // Pairs (candidate masks of 32 bits or less).  Two events whose candidate blocks are
  // NC or more rows or columns apart touch disjoint positions, so they can be updated
  // at once, one per half-wave, with the results of updating them in order.  The
  // relevant events are taken in order, greedily: event i shares a step with event i+1
  // when the two are disjoint and i does not already share one with i-1.  Bit i of D:
  // relevant events i and i+1 are disjoint; within each run of set bits the pairs start
  // at the run's first bit and every second bit after it, i.e. at the bits with the
  // parity of the run's start.
  const int lane = threadIdx.x & (kWave - 1);
  const uint64_t above = relm & ~((2ull << lane) - 1ull);  // relevant events after this one
  const int nxt = above ? __builtin_ctzll(above) : lane;
  const int oyn = __shfl(oy0, nxt), oxn = __shfl(ox0, nxt);
  const bool dis = rel && above != 0 && (abs(oyn - oy0) >= g.NC || abs(oxn - ox0) >= g.NC);
  // to lane = index among the relevant events (slot is a permutation of the lanes)
  const int dis_i = __builtin_amdgcn_ds_permute(slot << 2, dis ? 1 : 0);
  const uint64_t D = __ballot(dis_i != 0);
  constexpr uint64_t kEven = 0x5555555555555555ull;
  const uint64_t starts = D & ~(D << 1);
  // adding a run's start bit clears the run (the carry stops at the 0 after it)
  const uint64_t even_runs = D & ~(D + (starts & kEven));
  const uint64_t firsts = (even_runs & kEven) | (D & ~even_runs & ~kEven);
  const uint64_t seconds = firsts << 1;
  // relevant event i -> record 2 * step + half, step = i - (second events up to i)
  const int sec = (int)((seconds >> lane) & 1ull);
  const int place = 2 * (lane - lanes_below(seconds) - sec) + sec;
  const int rp = __shfl(place, slot);
  // every record of the chunk's steps covers nothing, then the events' (a wave's LDS
  // writes complete in order)
  c.rec[2 * lane] = make_int4(0, 0, 0, 0);
  c.rec[2 * lane + 1] = make_int4(0, 0, 0, 0);
  c.rec1[2 * lane] = make_int2(0, -1);
  c.rec1[2 * lane + 1] = make_int2(0, -1);
  if (rel) {
    c.rec[rp] = make_int4(tv, p0 * 4, q0 * 4, (int)(uint32_t)m);
    c.rec1[rp] = make_int2(0, idx);
  }
  return n - __popcll(seconds);
}

// The events of one decoded chunk, in order (salt_core/quant/scan.py:22-52 per update),
// with the spike ballots staged in LDS for the output (the work-group's merge, or the
// spike words of a row band).  M32: candidate masks fit 32 bits (NC^2 <= 32).  NOTRUNC:
// no position can hold max_queue_len events (max_queue_len >= the stream length), so
// every candidate event is a real queue column.  PAIR: n_ev steps of two events, one per
// half-wave (a step's second record covers nothing when it has one event).
template <int NIT, bool SAT, bool EXT, bool VTHN, bool M32, bool NOTRUNC, bool PAIR>
__device__ __forceinline__ void conv_events(const Quant& qz, const ConvLane& c,
                                            const int (&vtc)[NIT], int n_ev, int base,
                                            int& vmin_l, int& vmax_l) {
  const int lane = threadIdx.x & (kWave - 1);
  // The chunk's ballots and spike counts, indexed by the event's place in the chunk:
  // events without a candidate in this sub-band keep "no spike".  These clears precede
  // the events' entries (a wave's LDS writes complete in order).
#pragma unroll
  for (int it = 0; it < NIT; ++it) c.stg[lane * NIT + it] = ~0ull;
  c.wcnt[lane] = 0;
  if (n_ev == 0) return;
  constexpr bool kRec1 = !M32;  // the loop needs the second record word
  // lane e of sg_lo/sg_hi[it] collects event e's spike ballot; they are stored once per
  // chunk.
  uint32_t sg_lo[NIT], sg_hi[NIT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) { sg_lo[it] = ~0u; sg_hi[it] = ~0u; }
  const int fa = qz.fa, rc = qz.rc;
  const uint32_t nt1 = (uint32_t)c.ntab + 1u;
  const uint32_t lm32 = (uint32_t)c.lm;
  auto covers = [&](const int4& r, const int2& r1) -> bool {
    if (M32) return ((uint32_t)r.w & lm32) != 0u;
    return ((((uint64_t)(uint32_t)r1.x << 32) | (uint32_t)r.w) & c.lm) != 0;
  };
  // Software pipeline over two events.  LDS completes a wave's operations in order, so
  // a read issued after a write sees it: event e+1's registers, codes and decay code are
  // read right after event e has written its registers, and are waited for only when e+1
  // is updated -- one LDS round trip per event on the register chain.  Meanwhile event e
  // writes its positions' times, reads e+1's (after that write, so they are current) and
  // fetches the record of e+2.  NOTRUNC: the entries are last-update times alone (4 bytes;
  // the decode keeps the queue counts), so st.y is unused.
  auto tc_load = [&](int addr) -> int2 {
    return NOTRUNC ? make_int2(lds_ld<int32_t>(addr), 0) : lds_ld_tc(addr);
  };
  constexpr int kTcShift = NOTRUNC ? 0 : 1;  // record position base (bytes of a word) -> entry
  // An event's operands: register / code addresses and the values read there.
  struct Ops {
    int va, qa, A;
    int v[NIT], qv[NIT], vt[NIT], mnv[NIT], mxv[NIT];
  };
  // A position whose queue is full (max_queue_len real columns) drops the event and
  // its time (connectivity/conv.py:57-99 truncates the queue).
  auto act_of = [&](bool vc, const int2& st) { return NOTRUNC ? vc : (vc && st.y < c.mql); };
  // An event's base for this lane: the event's position base, or the spare base when
  // the lane has no candidate (NOTRUNC: also its register base, as every candidate
  // updates).
  auto base_of = [&](const int4& r, bool vc) { return vc ? r.y : c.sb; };
  auto read_ops = [&](Ops& o, const int4& r, int bse, bool vc, const int2& st) {
    const bool act = act_of(vc, st);
    // Decay code: dt = 0 -> identity, 1..n -> table, > n -> 0 (an unsigned clamp).
    o.A = lds_ld<int32_t>(c.extb + (int)(min((uint32_t)(r.x - st.x), nt1) << 2));
    o.va = (NOTRUNC ? bse : (act ? r.y : c.sb)) + c.lvb;
    o.qa = act ? r.z + c.lqb : c.q_zero_b;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      o.v[it] = lds_ld<int32_t>(o.va + it * c.GiVSb);
      o.qv[it] = lds_ld<int32_t>(o.qa + it * c.GiQSb);
      o.vt[it] = VTHN ? lds_ld<int32_t>(o.va + it * c.GiVSb + c.dth) : vtc[it];
      if (EXT) {
        o.mnv[it] = lds_ld<int32_t>(o.va + it * c.GiVSb + c.dmn);
        o.mxv[it] = lds_ld<int32_t>(o.va + it * c.GiVSb + c.dmx);
      }
    }
  };
  // this lane's record of step e: rec[RS * e + rh]
  constexpr int RS = PAIR ? 2 : 1;
  const int rh = PAIR ? c.rh : 0;
  int4 r = c.rec[rh];
  int2 r1 = kRec1 ? c.rec1[rh] : make_int2(0, 0);
  bool vc = covers(r, r1);
  int bse = base_of(r, vc);
  int pab = (bse << kTcShift) + c.ltb;  // this lane's (time, count) entry for the event
  int2 st = tc_load(pab);
  int4 rn = c.rec[RS + rh];  // records past the last step cover nothing
  int2 rn1 = kRec1 ? c.rec1[RS + rh] : make_int2(0, 0);
  Ops o;
  read_ops(o, r, bse, vc, st);
  // One event; everything carried becomes the next event's.
  auto event = [&](int e) {
    // this event's positions: time (and count), written by every lane of the position
    // (the slots of one candidate write the same entry with the same value)
    if (NOTRUNC)
      lds_st<int32_t>(pab, r.x);
    else
      lds_st_tc(pab, act_of(vc, st) ? r.x : st.x, st.y + 1);
    // the next event's positions, after that write
    const bool vcn = covers(rn, rn1);
    const int bsen = base_of(rn, vcn);
    const int pabn = (bsen << kTcShift) + c.ltb;
    const int2 stn = tc_load(pabn);
    const int4 rn2 = c.rec[RS * (e + 2) + rh];
    const int2 rn12 = kRec1 ? c.rec1[RS * (e + 2) + rh] : make_int2(0, 0);
    asm volatile("" ::: "memory");  // the reads above go out before this event's update
    uint64_t bal[NIT];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int32_t d = decay_mul_wide(o.v[it], o.A, fa, rc);
      const int32_t u = (int32_t)((uint32_t)d + (uint32_t)o.qv[it]);  // codes hold q*2^f_V
      const int32_t f = fit_bits<SAT>(u, qz);
      const bool keep = f < o.vt[it];
      lds_st<int32_t>(o.va + it * c.GiVSb, keep ? f : 0);
      vmin_l = min(vmin_l, u);
      vmax_l = max(vmax_l, u);
      if (EXT) {
        lds_st<int32_t>(o.va + it * c.GiVSb + c.dmn, min(o.mnv[it], u));
        lds_st<int32_t>(o.va + it * c.GiVSb + c.dmx, max(o.mxv[it], u));
      }
      // Staged as the lanes that kept their value (the others spiked): one compare.
      bal[it] = __ballot(keep);
    }
    asm volatile("" ::: "memory");  // the next event's reads come after these writes
    read_ops(o, rn, bsen, vcn, stn);
    // The ballots are staged here, after the next event's reads have gone out: the
    // lane index passes through an empty asm so that the compiler keeps the writes here
    // (issued earlier, they would wait for the compare).
    int el = e;
    asm volatile("" : "+s"(el));
#pragma unroll
    for (int it = 0; it < NIT; ++it) stage_to_lane(sg_lo[it], sg_hi[it], bal[it], el);
    r = rn;
    r1 = rn1;
    vc = vcn;
    st = stn;
    pab = pabn;
    rn = rn2;
    rn1 = rn12;
  };
  // Two events per iteration: one loop branch per pair, and the carried state need not
  // be copied between registers after every event.  The wave's priority steps down from
  // 3 to 0 over each quarter of the chunk: the waves of other streams sharing a SIMD are
  // at other points of their chunks, so the one furthest behind in its own chunk is
  // served first instead of the oldest wave, which would otherwise run ahead and leave
  // the younger ones to finish alone, latency-bound, at the end of the kernel.  PAIR
  // (chosen for grids under two work-groups per CU, where a SIMD has few waves to order)
  // keeps one priority: the steps cost more than they save there (measured).
  constexpr int kSegs = PAIR ? 1 : 4;
  int e = 0;
#pragma unroll
  for (int q = 0; q < kSegs; ++q) {
    if (!PAIR) {
      switch (q) {
        case 0: __builtin_amdgcn_s_setprio(3); break;
        case 1: __builtin_amdgcn_s_setprio(2); break;
        case 2: __builtin_amdgcn_s_setprio(1); break;
        default: __builtin_amdgcn_s_setprio(0); break;
      }
    }
    const int end = min(n_ev, (q + 1) * (kWave / kSegs));
    for (; e + 1 < end; e += 2) {
      event(e);
      event(e + 1);
    }
    if (e < end) event(e++);
  }
  if (!PAIR) __builtin_amdgcn_s_setprio(3);
  if (PAIR && lane < n_ev) {
    // step lane: half-wave h's ballot bits belong to the event of record 2 * lane + h
    const int j0 = c.rec1[2 * lane].y - base, j1 = c.rec1[2 * lane + 1].y;
    int n0 = 0, n1 = 0;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const uint64_t k0 = 0xffffffff00000000ull | sg_lo[it];
      const uint64_t k1 = 0xffffffff00000000ull | sg_hi[it];
      c.stg[j0 * NIT + it] = k0;
      n0 += __popcll(~k0);
      if (j1 >= 0) c.stg[(j1 - base) * NIT + it] = k1;
      n1 += __popcll(~k1);
    }
    c.wcnt[j0] = n0;
    if (j1 >= 0) c.wcnt[j1 - base] = n1;
  }
  if (!PAIR && lane < n_ev) {
    const int jc = c.rec1[lane].y - base;  // the event's index within the chunk
    int nsp = 0;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const uint64_t kept = ((uint64_t)sg_hi[it] << 32) | sg_lo[it];
      c.stg[jc * NIT + it] = kept;
      nsp += __popcll(~kept);
    }
    c.wcnt[jc] = nsp;
  }
}

// Catch-up column: decay to the last real input time T (connectivity/conv.py:102-125),
// then the final registers of this wave's ocn channels over its PW positions (rows of W,
// at row stride Wp in LDS).  An empty position's catch-up has dt = 0; the identity
// columns after it repeat V.  A full queue has no catch-up column.  Returns the largest
// per-position event count.
template <bool EXT, bool TSPLIT>
__device__ __forceinline__ int conv_finish(const Quant& qz, const ConvLane& c, int lane,
                                           int T, int ocn, int PW, int W, int Wp, int VS,
                                           size_t v_base, int HW, int32_t* v_final,
                                           int32_t* v_min, int32_t* v_max, int& vmin_l,
                                           int& vmax_l) {
  // (last-update time, queue count) of the position in LDS
  auto entry = [&](int pp) -> int2 {
    return TSPLIT ? make_int2(reinterpret_cast<const int32_t*>(c.tc)[pp], c.cnt[pp]) : c.tc[pp];
  };
  int maxcnt = 0;
  for (int i = lane; i < PW; i += kWave) maxcnt = max(maxcnt, entry((i / W) * Wp + i % W).y);
  for (int li = lane; li < ocn * PW; li += kWave) {
    const int s = li / PW;
    const int p = li - s * PW;
    const int pp = (p / W) * Wp + p % W;  // the position in LDS
    const int2 st = entry(pp);
    const int vi = s * VS + pp;
    int32_t vv = c.Vs[vi];
    int32_t mnn = EXT ? c.mn[vi] : 0, mxx = EXT ? c.mx[vi] : 0;
    if (st.y < c.mql) {
      const int dt = st.y > 0 ? T - st.x : 0;
      vv = decay_mul_wide(vv, c.ext[decay_slot(dt, c.ntab)], qz.fa, qz.rc);  // |D| <= |V|
      vmin_l = min(vmin_l, vv);
      vmax_l = max(vmax_l, vv);
      mnn = min(mnn, vv);
      mxx = max(mxx, vv);
    }
    const size_t ng = v_base + (size_t)s * HW + p;
    if (v_final) v_final[ng] = vv;
    if (EXT) {
      v_min[ng] = mnn;
      v_max[ng] = mxx;
    }
  }
  return wave_max(maxcnt);
}

template <int NIT, bool SAT, bool EXT, bool VTHN, bool M32, bool NOTRUNC, bool PAIR>
__global__ void __launch_bounds__(kWave * kConvBlockWaves) conv_layer_kernel(ConvArgs a) {
  extern __shared__ int32_t smem[];
  const ConvGeom& g = a.g;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int nthr = blockDim.x;
  // Waves [0, spw * nwps): wave wv serves stream slot ks of the work-group's spw streams,
  // as its channel-group wave wl.  Then one helper wave per (stream slot, sub-band), which
  // decodes the events and places every channel group's spikes.
  const int nwps = a.ncg * a.nsb;
  const int nch = a.spw * nwps;
  const bool helper = wv >= nch;
  const int hw = wv - nch;
  const int ks = helper ? hw / a.nsb : wv / nwps;
  const int wl = helper ? 0 : wv - ks * nwps;
  // Row-band plans: the bands of a stream read the same events, so they run on one XCD.
  const int n_wg = gridDim.x * gridDim.y;
  const int lin = blockIdx.y * gridDim.x + blockIdx.x;
  const int wg = a.merge ? lin : xcd_order(lin, n_wg);
  const int bx = wg % gridDim.x, by = wg / gridDim.x;  // (band, group of streams)
  const int b = by * a.spw + ks;
  const bool live = b < a.B;  // the last work-group's slots past the batch have no stream
  const int cg = wl % a.ncg;                        // channel group (helper: none, 0)
  const int sb = helper ? hw - ks * a.nsb : wl / a.ncg;  // sub-band
  const int Gi = a.Gi, Gp = NIT * a.Gi;
  const int oc0 = cg * a.G;
  const int ocn = max(0, min(a.G, g.OC - oc0));
  const int rows_end = min(g.H, bx * a.R + a.R);
  const int r0 = bx * a.R + sb * a.Rw;
  const int rn = max(0, min(a.Rw, rows_end - r0));
  const int W = g.W, Wp = g.Wp, PWs = a.Rw * Wp, PW = rn * W;
  const int ICKK = g.IC * g.K * g.K;
  const Quant& qz = a.qz;
  const int npos = conv_pos_words(PWs, g.NC2, conv_spare_pad(a.Rw, g.NC));
  const ConvLds lay = conv_lds_layout(qz.n_table, a.spw, a.ncg, a.nsb, Gp, NIT, a.VS, a.QS,
                                      PWs, npos, EXT, VTHN, NOTRUNC, PAIR);
  const int VS = lay.vs, QS = lay.qst;
  constexpr int RS = PAIR ? 2 : 1;  // records per step
  // regions: this (stream, sub-band)'s, the stream's sub-band 0's, this wave's (none for a
  // helper wave: it touches no per-wave array), and the stream's first wave's
  int32_t* const band = smem + lay.shared_words + (ks * a.nsb + sb) * lay.band_words;
  int32_t* const band0 = smem + lay.shared_words + ks * a.nsb * lay.band_words;
  int32_t* const wbase = smem + lay.waves + wv * lay.wave_words;
  const int32_t* const swave0 = smem + lay.waves + ks * nwps * lay.wave_words;
  int2* lanemap = reinterpret_cast<int2*>(smem + lay.lanemap);
  int32_t* red = smem + lay.red;
  int32_t* ext = smem + lay.ext;
  int4* const recs = reinterpret_cast<int4*>(band + lay.rec);
  int2* const recs1 = reinterpret_cast<int2*>(band + lay.rec1);
  int32_t* const nev = band + lay.nev;
  int2* const evt0 = reinterpret_cast<int2*>(band0 + lay.evt);
  uint64_t* const stgs = reinterpret_cast<uint64_t*>(wbase + lay.stg);
  ConvLane c;
  c.ext = ext;
  c.qs = smem + lay.qs + cg * Gp * QS;
  // The helper wave of a (stream, sub-band) decodes its events (and, NOTRUNC, keeps the
  // queue counts); the channel groups read its records.
  const bool dec = helper;
  c.tc = reinterpret_cast<int2*>(wbase + lay.tc);
  c.cnt = band + lay.cnt;
  int32_t* const cnt_kept = (NOTRUNC && dec) ? c.cnt : nullptr;
  int32_t* vthc = wbase + lay.vthc;
  c.Vs = wbase + lay.v;
  c.mn = wbase + lay.mn;
  c.mx = wbase + lay.mx;
  c.th = wbase + lay.th;

  // ---- shared state: decay table, ballot bit -> (slot, position offset), codes
  load_ext_table(ext, a.table, qz.n_table, qz.fa, tid, nthr);
  for (int k = tid; k < kWave; k += nthr) {
    const int s = k / g.NC2, cd = k - s * g.NC2;
    lanemap[k] = make_int2(s, (cd / g.NC) * W + (cd - (cd / g.NC) * g.NC));
  }
  for (int i = tid; i < a.ncg * Gp * QS; i += nthr) {
    const int gi = i / (Gp * QS), rem = i - gi * (Gp * QS);
    const int s = rem / QS, k = rem - s * QS;
    const int oc = gi * a.G + s;
    // Codes are stored pre-shifted, q * 2^f_V in two's complement (U = D + q*2^f_V).
    smem[lay.qs + i] = (s < a.G && oc < g.OC && k < ICKK)
                           ? (int32_t)((uint32_t)load_code_bits(a.q, (size_t)oc * ICKK + k,
                                                                a.q_bits) << qz.fV)
                           : 0;
  }
  // ---- this wave's state
  if (!helper) {
    for (int i = lane; i < Gp; i += kWave) {
      int v = INT_MAX;  // unreachable: registers stay below 2^29
      if (i < ocn) {
        if (qz.vth_kind == SALT_VTH_SCALAR) v = qz.vth_scalar;
        else if (qz.vth_kind == SALT_VTH_PER_CHANNEL) v = qz.vth[oc0 + i];
      }
      vthc[i] = v;
    }
    for (int i = lane; i < Gp * VS; i += kWave) {
      c.Vs[i] = 0;
      if (EXT) { c.mn[i] = 0; c.mx[i] = 0; }
      if (VTHN) {
        const int s = i / VS, p = i - s * VS, row = p / Wp, col = p - row * Wp;
        c.th[i] = (s < ocn && row < rn && col < W)
                      ? qz.vth[(size_t)(oc0 + s) * g.HW + (r0 + row) * W + col]
                      : INT_MAX;
      }
    }
    for (int i = lane; i < (NOTRUNC ? 1 : 2) * lay.tcn; i += kWave) wbase[lay.tc + i] = 0;
  } else {
    if (NOTRUNC)
      for (int i = lane; i < PWs; i += kWave) c.cnt[i] = 0;
    if (lane < 2 * RS)  // the records after a full chunk: no candidate
      for (int bf = 0; bf < kConvRecBufs; ++bf) {
        recs[bf * conv_recs(PAIR) + RS * kWave + lane] = make_int4(0, 0, 0, 0);
        recs1[bf * conv_recs(PAIR) + RS * kWave + lane] = make_int2(0, -1);
      }
  }

  conv_lane_setup(c, g, lane, Gi, VS, QS, PWs, oc0, qz.n_table, NOTRUNC ? 4 : 8, smem, PAIR);
  int vtc[NIT];

  const int L = a.L;
  auto real_count = [&](int bi) {
    const int nr = bi < a.B ? a.n_real[bi] : 0;
    return nr < 0 ? 0 : (nr < L ? nr : L);
  };
  const int n_eff = real_count(b);
  // Row-band plans with event lists: this work-group's events are its list's entries.
  const int32_t* lst = nullptr;
  int n_list = 0;
  if (a.blist && live) {
    const int bi = b * gridDim.x + bx;
    n_list = __builtin_amdgcn_readfirstlane(a.bcnt[bi]);
    lst = a.blist + (size_t)b * a.bcap + a.boff[bi];
  }
  // The chunk loop runs to the work-group's longest stream (or list), so that every wave
  // meets every barrier; a stream's chunks past its own events decode to no events.
  int n_grp = 0;
  if (a.blist) {
    n_grp = n_list;
  } else {
    for (int i = lane; i < a.spw; i += kWave)
      n_grp = max(n_grp, real_count(by * a.spw + i));
    n_grp = __builtin_amdgcn_readfirstlane(wave_max(n_grp));
  }
  const int nchunks = (n_grp + kWave - 1) / kWave;
  const float* tb = a.times + (size_t)(live ? b : 0) * L;
  const int32_t* sb_src = a.src + (size_t)(live ? b : 0) * L;

  int vmin_l = 0, vmax_l = 0;
  int out_base = 0;  // spikes of the stream emitted so far (merge mode)

  // Next chunk of events, loaded one chunk ahead and converted only when its chunk is
  // decoded, so the loads' latency is covered by a chunk of work.  The index is clamped
  // into the stream (entries past n_eff are not real: conv_decode checks j < n_eff);
  // a stream without events loads nothing.
  const int jl = n_eff - 1;
  float t_n = 0.0f;
  int s_n = -1;
  // With a list: the original indices of the next chunk's events (jo_n) and of the one
  // after (jo_nn), the index loaded two chunks ahead and the event one chunk ahead.
  int jo_n = 0, jo_nn = 0;
  if (dec) {
    if (a.blist) {
      if (n_list > 0) {
        jo_n = lst[min(lane, n_list - 1)];
        jo_nn = lst[min(kWave + lane, n_list - 1)];
        t_n = tb[jo_n];
        s_n = sb_src[jo_n];
      }
    } else if (jl >= 0) {
      t_n = tb[min(lane, jl)];
      s_n = sb_src[min(lane, jl)];
    }
  }
  // Decoding wave: chunk k into record buffer k % 2 (and, sub-band 0, into event buffer
  // k % 3: merge mode the chunk's event times and plane positions, row bands the events'
  // stream indices).
  auto decode = [&](int k) {
    const int bf = k & 1;
    const int idx = k * kWave + lane;  // place in the stream or the band's list
    int j = idx;
    const int tv = time_ms(t_n), sv = s_n;
    if (a.blist) {
      // list position -> original index (past the list: not real)
      j = j < n_list ? jo_n : n_eff;
      if (n_list > 0) {
        t_n = tb[jo_nn];
        s_n = sb_src[jo_nn];
        jo_n = jo_nn;
        jo_nn = lst[min((k + 2) * kWave + lane, n_list - 1)];
      }
    } else if (jl >= 0) {
      const int j2 = min(j + kWave, jl);
      t_n = tb[j2];
      s_n = sb_src[j2];
    }
    c.rec = recs + bf * conv_recs(PAIR);
    c.rec1 = recs1 + bf * conv_recs(PAIR);
    int oy0 = 0, ox0 = 0;
    const int n = conv_decode<PAIR>(g, c, tv, sv, j, idx, n_eff, r0, rn, oy0, ox0, cnt_kept);
    if (lane == 0) nev[bf] = n;
    if (sb == 0)
      evt0[(k % kConvEvtBufs) * kWave + lane] =
          a.merge ? make_int2(tv, oy0 * W + ox0) : make_int2(j, 0);
  };
  // Row bands, the helper wave: for each event of chunk k with a spike in the band, every
  // channel group's spike words (all NIT, spikes or not) in the event's slot for this
  // band; it marks the slot valid and adds the event's spikes in the band to its
  // compaction segment.  Lane = the event's index in the chunk.
  const int slot = bx % max(a.nslots, 1);
  auto store_words = [&](int k) {
    const int bf = k & 1;
    int tot = 0;
    for (int g2 = 0; g2 < a.ncg; ++g2)  // one sub-band per row band
      tot += swave0[g2 * lay.wave_words + lay.wcnt + bf * kWave + lane];
    if (tot == 0) return;
    const int jj = evt0[(k % kConvEvtBufs) * kWave + lane].x;
    const size_t ev = (size_t)b * L + jj;
    uint64_t* const w = a.words + (ev * a.nslots + slot) * (size_t)(a.ncg * NIT);
    for (int g2 = 0; g2 < a.ncg; ++g2) {
      const uint64_t* const kept = reinterpret_cast<const uint64_t*>(
          swave0 + g2 * lay.wave_words + lay.stg) + bf * kWave * NIT + lane * NIT;
#pragma unroll
      for (int it = 0; it < NIT; ++it) w[g2 * NIT + it] = ~kept[it];
    }
    atomicOr(&a.valid[ev], 1u << slot);
    atomicAdd(&a.seg_cnt[(size_t)b * a.nseg + jj / kCompactSeg], tot);
  };
  // Merge mode: the sub-band's spikes of chunk k in channel groups [g_begin, g_end), at
  // their places in the stream's output, ordered (event, channel group, iteration, bit) =
  // (event, ascending neuron id) -- the order of salt_core/stream.py:24-46; the helper
  // wave places every group's (hwalk), or each channel-group wave its own.  Lane = the
  // event's index in the chunk.  An event's spikes start after those of the chunk's
  // earlier events (a scan of the stream's waves' counts) and, within it, after the lower
  // channel groups' spikes and the group's lower iterations and bits; the sub-bands'
  // ballots of one channel group are disjoint and share the lane mapping, so the bits
  // below a spike are counted in their union.
  auto walk = [&](int k, int g_begin, int g_end) {
    const int bf = k & 1;
    auto count = [&](int s2, int g2) {  // wave s2 * ncg + g2: sub-band s2, channel group g2
      return swave0[(s2 * a.ncg + g2) * lay.wave_words + lay.wcnt + bf * kWave + lane];
    };
    int tot = 0, before = 0;
    for (int s2 = 0; s2 < a.nsb; ++s2)
      for (int g2 = 0; g2 < a.ncg; ++g2) {
        const int cw = count(s2, g2);
        tot += cw;
        before += g2 < g_begin ? cw : 0;
      }
    if (__ballot(tot != 0) == 0) return;  // no spike in the chunk
    const int incl = wave_incl_scan(tot);
    const int total = __builtin_amdgcn_readlane(incl, kWave - 1);
    const int2 ev = evt0[(k % kConvEvtBufs) * kWave + lane];  // read with every lane active
    const float te = ms_time(ev.x);
    int pos = out_base + (incl - tot) + before;
    for (int g2 = g_begin; g2 < g_end; ++g2) {
      const uint64_t* const stg_cg = reinterpret_cast<const uint64_t*>(
          swave0 + g2 * lay.wave_words + lay.stg) + bf * kWave * NIT + lane * NIT;
      const int oc0g = g2 * a.G;
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        uint64_t all = 0, mine = 0;
        for (int s2 = 0; s2 < a.nsb; ++s2) {
          const uint64_t v = ~stg_cg[s2 * a.ncg * (lay.wave_words / 2) + it];
          all |= v;
          mine = s2 == sb ? v : mine;
        }
        while (mine) {
          const int kb = __builtin_ctzll(mine);
          mine &= mine - 1;
          const int p = pos + __popcll(all & ((1ull << kb) - 1));
          const int2 lmk = lanemap[kb];
          const int oc = oc0g + it * Gi + lmk.x;
          if (p < a.cap) {
            a.out_t[(size_t)b * a.cap + p] = te;
            a.out_s[(size_t)b * a.cap + p] = oc * g.HW + ev.y + lmk.y;
          }
        }
        pos += __popcll(all);
      }
    }
    out_base += total;
  };

  if (dec && nchunks > 0) decode(0);
  __syncthreads();
  if (!helper) {
#pragma unroll
    for (int it = 0; it < NIT; ++it) vtc[it] = vthc[min(it * Gi + c.oc_lane - oc0, Gp - 1)];
  }
  // One barrier per chunk: chunk k's records and counts were written before the last
  // barrier; the next chunk's decode writes the other record buffer, whose readers
  // finished before it; the walk of chunk k-1 reads the ballots and counts written
  // before it (the channel groups write chunk k's into the other buffers meanwhile), and
  // event info decoded two chunks before the next decode's.
  // A helper with heavy per-chunk work is served before the channel-group waves at their
  // lowest priority, so its stream does not wait for it at the chunk barrier.
  if (helper && a.hprio) __builtin_amdgcn_s_setprio(1);
  for (int k = 0; k < nchunks; ++k) {
    const int bf = k & 1;
    if (helper) {
      if (k + 1 < nchunks) decode(k + 1);
      if (k > 0) {
        if (!a.merge) {
          if (live) store_words(k - 1);
        } else if (a.hwalk) {
          walk(k - 1, 0, a.ncg);
        }
      }
    } else {
      if (k > 0 && a.merge && !a.hwalk) walk(k - 1, cg, cg + 1);
      c.rec = recs + bf * conv_recs(PAIR);
      c.rec1 = recs1 + bf * conv_recs(PAIR);
      const int n_ev = __builtin_amdgcn_readfirstlane(nev[bf]);
      c.stg = stgs + bf * kWave * NIT;
      c.wcnt = wbase + lay.wcnt + bf * kWave;
      conv_events<NIT, SAT, EXT, VTHN, M32, NOTRUNC, PAIR>(qz, c, vtc, n_ev, k * kWave,
                                                           vmin_l, vmax_l);
    }
    __syncthreads();
  }
  if (nchunks > 0) {
    if (helper) {
      if (!a.merge) {
        if (live) store_words(nchunks - 1);
      } else if (a.hwalk) {
        walk(nchunks - 1, 0, a.ncg);
      }
    } else if (a.merge && !a.hwalk) {
      walk(nchunks - 1, cg, cg + 1);
    }
  }

  const int T = n_eff > 0 ? time_ms(tb[n_eff - 1]) : 0;
  int maxcnt = 0;
  if (live && !helper)
    maxcnt = conv_finish<EXT, NOTRUNC>(qz, c, lane, T, ocn, PW, W, Wp, VS,
                                   (size_t)b * (g.OC * g.HW) + (size_t)oc0 * g.HW + r0 * W,
                                   g.HW, a.v_final, a.v_min, a.v_max, vmin_l, vmax_l);
  vmin_l = wave_min(vmin_l);
  vmax_l = wave_max(vmax_l);
  if (lane == 0) {
    red[wv * 4 + 0] = vmin_l;
    red[wv * 4 + 1] = vmax_l;
    red[wv * 4 + 2] = maxcnt;
  }
  __syncthreads();
  if (!live) return;
  // merge mode: the stream's spike count and pads, by a wave that placed spikes (every
  // such wave counts all of them): sub-band 0's helper, or the first channel group
  if (a.merge && (a.hwalk ? helper && sb == 0 : wl == 0 && !helper)) {
    if (lane == 0) a.out_n[b] = out_base;
    if (a.fill_pads)
      for (int i = min(out_base, a.cap) + lane; i < a.cap; i += kWave) {
        a.out_t[(size_t)b * a.cap + i] = kPadTime;
        a.out_s[(size_t)b * a.cap + i] = 0;
      }
  }
  if (helper || wl != 0) return;
  for (int w = wv + 1; w < wv + nwps; ++w) {  // the stream's other channel-group waves
    vmin_l = min(vmin_l, red[w * 4 + 0]);
    vmax_l = max(vmax_l, red[w * 4 + 1]);
    maxcnt = max(maxcnt, red[w * 4 + 2]);
  }
  const int ovf = (vmin_l < -qz.half || vmax_l > qz.half - 1) ? 1 : 0;
  if (a.merge) {
    if (lane == 0) {
      a.stats[b * 4 + 0] = vmin_l;
      a.stats[b * 4 + 1] = vmax_l;
      a.stats[b * 4 + 2] = maxcnt + 1;
      a.stats[b * 4 + 3] = ovf;
    }
  } else if (lane == 0) {
    atomicMin(&a.stats[b * 4 + 0], vmin_l);
    atomicMax(&a.stats[b * 4 + 1], vmax_l);
    atomicMax(&a.stats[b * 4 + 2], maxcnt + 1);
    atomicOr(&a.stats[b * 4 + 3], ovf);
  }
}

}  // namespace salt
