// libsalt_hip.so: MI355X (gfx950, CDNA4) kernels and C-ABI for the integer
// event-by-event forward pass of salt_core/quant.  The exported entry points are
// declared, with their reference counterparts, in include/salt_hip.h.
//
// Work decomposition.  A stream is strictly sequential per neuron, so parallelism
// comes from streams (batch) and from the neurons one event touches.  Each layer is
// split into partitions and one 64-lane wavefront owns one (stream, partition) pair,
// consuming that stream's events in order (conv_kernel.hpp, fc_kernel.hpp):
//   conv: partition = a group of output channels x a band of output rows, state in LDS;
//   FC:   partition = a slice of 64*NPL neurons, state in VGPRs.
// When one partition holds the whole layer the wave writes the spike stream itself:
// spikes of one event come out lane-ordered, which is ascending neuron id, the order
// of salt_core/stream.py:29-30.  Otherwise each partition sets per-event spike bits
// (bit order = neuron order) and compact_kernel turns them into the stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>

#include "launch.hpp"
#include "trace_kernel.hpp"

using namespace salt;

namespace {

// ------------------------------------------------------------------ errors

thread_local std::string g_err;

int32_t fail(int32_t code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define HIP_TRY(expr)                                                          \
  do {                                                                         \
    hipError_t e_ = (expr);                                                    \
    if (e_ != hipSuccess)                                                      \
      return fail(-2, "%s failed: %s", #expr, hipGetErrorString(e_));          \
  } while (0)

// LDS per row-band work-group: half a CU's, so two work-groups share a CU with bands as
// tall as that allows (measured on configuration 4, conv kernel per launch: 52 KiB
// 3.44 ms, 64 KiB 2.87 ms, 80 KiB 2.63 ms, 100 KiB 3.94 ms).
constexpr int kLdsBandBudget = kLdsMax / 2;
constexpr int kMaxTable = 1 << 20;           // decay-table entries (times stay exact)

__global__ void fill_i32_kernel(int32_t* p, int32_t value, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = value;
}

// ------------------------------------------------------------------ compaction

// Spikes -> ordered stream, in segments of kCompactSeg events so that a stream's walk and
// its padding spread over many waves.  One wave per (segment, stream) starts its part of
// the stream after the earlier segments' spikes, from per-segment spike counts (kept by
// the conv kernel, or counted by compact_count_kernel for FC slices), and reads nothing
// of a segment without spikes.  Walking the spikes of an event in ascending neuron id
// gives the (event, neuron) order of salt_core/stream.py:24-46.

int compact_segments(int L) { return std::max(1, (L + kCompactSeg - 1) / kCompactSeg); }

__device__ __forceinline__ int stream_events(const int32_t* n_real, int b, int L) {
  const int nr = n_real[b];
  return nr < 0 ? 0 : (nr < L ? nr : L);
}

// Segment s's first place in stream b's output (before) and the stream's spike count.
__device__ __forceinline__ void segment_start(const int32_t* seg_cnt, int b, int nseg, int s,
                                              int& before, int& all) {
  const int lane = threadIdx.x & (kWave - 1);
  before = 0;
  all = 0;
  for (int t = lane; t < nseg; t += kWave) {
    const int c = seg_cnt[b * nseg + t];
    before += t < s ? c : 0;
    all += c;
  }
  before = __builtin_amdgcn_readlane(wave_incl_scan(before), kWave - 1);
  all = __builtin_amdgcn_readlane(wave_incl_scan(all), kWave - 1);
}

// The stream's count (by the last segment's wave) and its padding, shared by the
// segments' waves: entries past the spikes hold (1e12, 0) when fill_pads.
__device__ __forceinline__ void segment_finish(int b, int s, int nseg, int all, int cap,
                                               int fill_pads, float* out_t, int32_t* out_s,
                                               int32_t* out_n) {
  const int lane = threadIdx.x & (kWave - 1);
  if (s == nseg - 1 && lane == 0) out_n[b] = all;
  if (fill_pads)
    for (int i = min(all, cap) + s * kWave + lane; i < cap; i += nseg * kWave) {
      out_t[(size_t)b * cap + i] = kPadTime;
      out_s[(size_t)b * cap + i] = 0;
    }
}

// FC slices: one bit per (event, neuron), words in neuron order (neuron = word*32 + bit).
struct CompactArgs {
  int words, L;
  const float* times;
  const int32_t* n_real;
  const uint32_t* masks;
  int cap, fill_pads;
  float* out_t;
  int32_t* out_s;
  int32_t* out_n;
};

// Spikes per (stream, segment): the segment's mask words as one flat, coalesced array.
__global__ void __launch_bounds__(64) compact_count_kernel(CompactArgs a, int32_t* seg_cnt,
                                                           int nseg) {
  const int lane = threadIdx.x;
  const int s = blockIdx.x, b = blockIdx.y;
  const int n_eff = stream_events(a.n_real, b, a.L);
  const int j0 = min(n_eff, s * kCompactSeg), j1 = min(n_eff, j0 + kCompactSeg);
  const uint32_t* m = a.masks + ((size_t)b * a.L + j0) * a.words;
  const size_t nw = (size_t)(j1 - j0) * a.words;
  int cnt = 0;
  for (size_t i = lane; i < nw; i += kWave) cnt += __popc(m[i]);
  const int total = __builtin_amdgcn_readlane(wave_incl_scan(cnt), kWave - 1);
  if (lane == 0) seg_cnt[b * nseg + s] = total;
}

// One wave per (segment, stream); lane = event within a window of 64.
__global__ void __launch_bounds__(64) compact_kernel(CompactArgs a, const int32_t* seg_cnt,
                                                     int nseg) {
  const int lane = threadIdx.x;
  const int s = blockIdx.x, b = blockIdx.y;
  const int L = a.L;
  const int n_eff = stream_events(a.n_real, b, L);
  int before, all;
  segment_start(seg_cnt, b, nseg, s, before, all);
  int out_base = before;
  const int j_end = seg_cnt[b * nseg + s] > 0 ? min(n_eff, (s + 1) * kCompactSeg) : 0;
  for (int base = s * kCompactSeg; base < j_end; base += kWave) {
    const int j = base + lane;
    const bool ok = j < j_end;
    const uint32_t* m = a.masks + ((size_t)b * L + j) * a.words;
    int count = 0;
    if (ok)
      for (int w = 0; w < a.words; ++w) count += __popc(m[w]);
    const int incl = wave_incl_scan(count);
    const int total = __builtin_amdgcn_readlane(incl, kWave - 1);
    if (ok && count > 0) {
      int pos = out_base + incl - count;
      const float te = a.times[(size_t)b * L + j];
      for (int w = 0; w < a.words; ++w)
        for (uint32_t bits = m[w]; bits; bits &= bits - 1) {
          if (pos < a.cap) {
            a.out_t[(size_t)b * a.cap + pos] = te;
            a.out_s[(size_t)b * a.cap + pos] = w * 32 + __builtin_ctz(bits);
          }
          ++pos;
        }
    }
    out_base += total;
  }
  segment_finish(b, s, nseg, all, a.cap, a.fill_pads, a.out_t, a.out_s, a.out_n);
}

// Conv row bands: the spike words of conv_layer_kernel (per event, one slot per band it
// reaches, valid bits telling which slots were stored).  Word (g, it) of a slot holds, at
// bit l, channel g*G + it*Gi + l / NC2 and candidate l % NC2 of the event's NC x NC grid;
// the slots of one event cover disjoint candidate rows, so a channel's candidates are the
// union of its bits over the stored slots.
struct BandCompactArgs {
  int L, HW, W, HWin, Win, K, S, P, NC, NC2, OC;
  int G, Gi, nit, ncg, nslots;
  const float* times;
  const int32_t* src;
  const int32_t* n_real;
  const uint64_t* words;
  const uint32_t* valid;
  int cap, fill_pads;
  float* out_t;
  int32_t* out_s;
  int32_t* out_n;
};

// One wave per (segment, stream); lane = event within a window of 64.
__global__ void __launch_bounds__(64) band_compact_kernel(BandCompactArgs a,
                                                          const int32_t* seg_cnt, int nseg) {
  const int lane = threadIdx.x;
  const int s = blockIdx.x, b = blockIdx.y;
  const int L = a.L;
  const int n_eff = stream_events(a.n_real, b, L);
  int before, all;
  segment_start(seg_cnt, b, nseg, s, before, all);
  int out_base = before;
  const int wpe = a.ncg * a.nit;  // words per (event, slot)
  const uint64_t cand_mask = a.NC2 >= 64 ? ~0ull : (1ull << a.NC2) - 1;
  const int j_end = seg_cnt[b * nseg + s] > 0 ? min(n_eff, (s + 1) * kCompactSeg) : 0;
  for (int base = s * kCompactSeg; base < j_end; base += kWave) {
    const int j = base + lane;
    const size_t ev = (size_t)b * L + j;
    const uint32_t vb = j < j_end ? a.valid[ev] : 0u;
    const uint64_t* const wv = a.words + ev * a.nslots * wpe;
    int count = 0;
    for (int sl = 0; sl < a.nslots; ++sl)
      if ((vb >> sl) & 1u)
        for (int w = 0; w < wpe; ++w) count += __popcll(wv[sl * wpe + w]);
    const int incl = wave_incl_scan(count);
    const int total = __builtin_amdgcn_readlane(incl, kWave - 1);
    if (count > 0) {
      int pos = out_base + incl - count;
      const float te = a.times[ev];
      const int rem = a.src[ev] % a.HWin;
      const int y = rem / a.Win, x = rem - (rem / a.Win) * a.Win;
      const int oy0 = floordiv_pos(y + a.P - a.K + a.S, a.S);
      const int ox0 = floordiv_pos(x + a.P - a.K + a.S, a.S);
      for (int oc = 0; oc < a.OC; ++oc) {
        const int g = oc / a.G, sc = oc - g * a.G, it = sc / a.Gi;
        const int wi = g * a.nit + it, sh = (sc - it * a.Gi) * a.NC2;
        uint64_t m = 0;
        for (int sl = 0; sl < a.nslots; ++sl)
          if ((vb >> sl) & 1u) m |= wv[sl * wpe + wi] >> sh;
        for (m &= cand_mask; m; m &= m - 1) {
          const int r = __builtin_ctzll(m);
          const int dy = r / a.NC, dx = r - (r / a.NC) * a.NC;
          if (pos < a.cap) {
            a.out_t[(size_t)b * a.cap + pos] = te;
            a.out_s[(size_t)b * a.cap + pos] = oc * a.HW + (oy0 + dy) * a.W + (ox0 + dx);
          }
          ++pos;
        }
      }
    }
    out_base += total;
  }
  segment_finish(b, s, nseg, all, a.cap, a.fill_pads, a.out_t, a.out_s, a.out_n);
}

// ------------------------------------------------------------------ row-band event lists

// Row-band plans: for every (stream, band of R output rows) the events whose candidate
// rows [ceil((y+P-K+1)/S), floor((y+P)/S)] meet the band (the decode's row test; it
// keeps a superset of the events with a candidate there), as original indices in order,
// so that a band's work-group decodes its events alone instead of the whole stream.
// Three small kernels, each event read once per pass: band_count_kernel counts the
// events of every band per segment of kBandSeg events, band_scan_kernel turns the counts
// into list positions, band_fill_kernel writes the lists.
constexpr int kBandSeg = 1024;    // events per segment of the list build
constexpr int kBandMaxRb = 4096;  // bands per stream with lists (LDS of the list build)
static_assert(kBandMaxRb * 12 <= 64 * 1024, "band_fill_kernel's LDS");

struct BandArgs {
  int L, R, H, n_rb, K, S, P, HWin, Win, n_src, cap, nseg;
  float rHWin, rWin, rS, rR;
  const int32_t* src;
  const int32_t* n_real;
  int32_t* cnt;      // [B][n_rb]: events in the band's list
  int32_t* off;      // [B][n_rb]: first entry of the band's list in the stream's region
  int32_t* list;     // [B][cap]
  int32_t* seg_pos;  // [B][nseg][n_rb]: counts per segment, then the segment's first places
};

// The bands [b0, b1] that source s (an input pixel) reaches: its candidate rows clipped to
// the plane, in bands of R rows; b1 < b0 when it reaches none (s < 0: no event).
__device__ __forceinline__ void band_range(const BandArgs& a, int s, int& b0, int& b1) {
  b0 = 0;
  b1 = -1;
  if (s < 0) return;
  s = min(s, a.n_src - 1);
  int ch, y, lo, hi;
  if (a.n_src <= (1 << 22)) {
    ch = div_small(s, a.HWin, a.rHWin);
    y = div_small(s - ch * a.HWin, a.Win, a.rWin);
    lo = div_small(y + a.P - a.K + a.S + a.K * a.S, a.S, a.rS) - a.K;
    hi = div_small(y + a.P, a.S, a.rS);
  } else {
    ch = s / a.HWin;
    y = (s - ch * a.HWin) / a.Win;
    lo = floordiv_pos(y + a.P - a.K + a.S, a.S);
    hi = (y + a.P) / a.S;
  }
  lo = max(lo, 0);
  hi = min(hi, a.H - 1);
  if (lo > hi) return;
  b0 = div_small(lo, a.R, a.rR);
  b1 = div_small(hi, a.R, a.rR);
}

__device__ __forceinline__ int band_events(const BandArgs& a, int b) {
  return stream_events(a.n_real, b, a.L);
}

// One wave per (segment, stream): the segment's events per band.
__global__ void __launch_bounds__(64) band_count_kernel(BandArgs a) {
  __shared__ int32_t hist[kBandMaxRb];
  const int lane = threadIdx.x;
  const int sg = blockIdx.x, b = blockIdx.y;
  for (int i = lane; i < a.n_rb; i += kWave) hist[i] = 0;
  __syncthreads();
  const int j0 = sg * kBandSeg, j1 = min(band_events(a, b), j0 + kBandSeg);
  const int32_t* src = a.src + (size_t)b * a.L;
  for (int base = j0; base < j1; base += kWave) {
    const int j = base + lane;
    int b0, b1;
    band_range(a, j < j1 ? src[j] : -1, b0, b1);
    for (int k = b0; k <= b1; ++k) atomicAdd(&hist[k], 1);
  }
  __syncthreads();
  int32_t* const out = a.seg_pos + ((size_t)b * a.nseg + sg) * a.n_rb;
  for (int i = lane; i < a.n_rb; i += kWave) out[i] = hist[i];
}

// One wave per stream, lane = band: each band's list length and offset (its stream's
// earlier bands' lengths), then each segment's first place in the band's list.
__global__ void __launch_bounds__(64) band_scan_kernel(BandArgs a) {
  const int lane = threadIdx.x;
  const int b = blockIdx.x;
  int32_t* const rows = a.seg_pos + (size_t)b * a.nseg * a.n_rb;
  constexpr int kBatch = 8;  // loads in flight per lane
  int run = 0;
  for (int rb0 = 0; rb0 < a.n_rb; rb0 += kWave) {
    const int rb = rb0 + lane;
    const bool ok = rb < a.n_rb;
    int tot = 0;
    for (int s0 = 0; s0 < a.nseg; s0 += kBatch) {
      int c[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        c[u] = (ok && s0 + u < a.nseg) ? rows[(size_t)(s0 + u) * a.n_rb + rb] : 0;
#pragma unroll
      for (int u = 0; u < kBatch; ++u) tot += c[u];
    }
    const int incl = wave_incl_scan(tot);
    int pos = run + incl - tot;
    if (ok) {
      a.cnt[b * a.n_rb + rb] = tot;
      a.off[b * a.n_rb + rb] = pos;
    }
    run += __builtin_amdgcn_readlane(incl, kWave - 1);
    for (int s0 = 0; s0 < a.nseg; s0 += kBatch) {
      int c[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        c[u] = (ok && s0 + u < a.nseg) ? rows[(size_t)(s0 + u) * a.n_rb + rb] : 0;
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        if (ok && s0 + u < a.nseg) rows[(size_t)(s0 + u) * a.n_rb + rb] = pos;
        pos += c[u];
      }
    }
  }
}

// One wave per (segment, stream): the segment's events appended to the lists of the
// bands they reach.  Per window of 64 events (lane = event): every lane marks its bit in
// the lane set of each band it reaches (an LDS OR), so that a lane's place in a band's
// list is the band's next place plus the lanes below it in the band's set; the lowest
// lane of each set then advances the band's next place and clears the set.  nslots:
// bands one event reaches at most.  LDS: n_rb lane sets (8 bytes) and next places.
__global__ void __launch_bounds__(64) band_fill_kernel(BandArgs a, int nslots) {
  extern __shared__ int32_t bsm[];
  uint64_t* const lanes_of = reinterpret_cast<uint64_t*>(bsm);
  int32_t* const next = bsm + 2 * a.n_rb;
  const int lane = threadIdx.x;
  // The segments of a stream run on one XCD: their partial lines of a band's list then
  // meet in one L2 before they reach HBM.
  const int wg = xcd_order(blockIdx.y * gridDim.x + blockIdx.x, gridDim.x * gridDim.y);
  const int sg = wg % gridDim.x, b = wg / gridDim.x;
  const int32_t* pos = a.seg_pos + ((size_t)b * a.nseg + sg) * a.n_rb;
  for (int i = lane; i < a.n_rb; i += kWave) {
    next[i] = pos[i];
    lanes_of[i] = 0;
  }
  __syncthreads();
  const int j0 = sg * kBandSeg, j1 = min(band_events(a, b), j0 + kBandSeg);
  const int32_t* src = a.src + (size_t)b * a.L;
  int32_t* const out = a.list + (size_t)b * a.cap;
  const uint64_t below = (1ull << lane) - 1;
  for (int base = j0; base < j1; base += kWave) {
    const int j = base + lane;
    int b0, b1;
    band_range(a, j < j1 ? src[j] : -1, b0, b1);
    for (int k = 0; k < nslots; ++k)
      if (b0 + k <= b1) atomicOr(reinterpret_cast<unsigned long long*>(&lanes_of[b0 + k]),
                                 1ull << lane);
    __syncthreads();
    uint32_t lead = 0;  // bit k: this lane is the lowest of band b0 + k's set
    for (int k = 0; k < nslots; ++k) {
      if (b0 + k > b1) continue;
      const uint64_t m = lanes_of[b0 + k];
      const int at = next[b0 + k];
      out[at + __popcll(m & below)] = j;
      lead |= (m & below) == 0 ? 1u << k : 0u;
    }
    __syncthreads();
    for (int k = 0; k < nslots; ++k) {
      if (!((lead >> k) & 1)) continue;
      const int bk = b0 + k;
      next[bk] += __popcll(lanes_of[bk]);
      lanes_of[bk] = 0;
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------ hash

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__global__ void __launch_bounds__(256) stream_hash_kernel(const float* t, const int32_t* s,
                                                          const int32_t* n, int cap,
                                                          uint64_t* out) {
  __shared__ uint64_t part[256];
  const int b = blockIdx.x;
  const int nb = n[b];
  const int m = nb < cap ? nb : cap;
  uint64_t acc = 0;
  for (int i = threadIdx.x; i < m; i += blockDim.x) {
    const uint32_t tb = __float_as_uint(t[(size_t)b * cap + i]);
    const uint64_t key = ((uint64_t)tb << 32) | (uint32_t)s[(size_t)b * cap + i];
    acc += mix64(mix64((uint64_t)i) ^ key);
  }
  part[threadIdx.x] = acc;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) part[threadIdx.x] += part[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0)
    out[b] = mix64(part[0] + (uint64_t)(uint32_t)nb * 0x2545F4914F6CDD1Dull);
}

// ------------------------------------------------------------------ transpose

template <typename T>
__global__ void transpose_kernel(const T* in, T* out, int n_out, int n_in) {
  // in: (n_out, n_in) -> out: (n_in, n_out)
  __shared__ T tile[32][33];
  const int bx = blockIdx.x * 32, by = blockIdx.y * 32;  // bx over n_in, by over n_out
  const int tx = threadIdx.x, ty = threadIdx.y;          // 32 x 8
  for (int r = ty; r < 32; r += 8) {
    const int o = by + r, i = bx + tx;
    if (o < n_out && i < n_in) tile[r][tx] = in[(size_t)o * n_in + i];
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    const int i = bx + r, o = by + tx;
    if (o < n_out && i < n_in) out[(size_t)i * n_out + o] = tile[tx][r];
  }
}

// ------------------------------------------------------------------ planning

struct ConvPlan {
  int H, W, HW, NC, NC2, Gi, G, nit, ncg, nsb, Rw, R, n_rb, merge, spw;
  int Wp, VS, QS;  // LDS row stride and slot strides (choose_layout)
  int tsplit;      // no queue truncation possible: times and counts in separate arrays
  int pair;        // two events per step, one per half-wave (NC2 <= 32)
  size_t lds;
};

int round_nit(int n) {  // smallest instantiated iteration count >= n
  if (n <= 4) return n < 1 ? 1 : n;
  return n <= 8 ? 8 : -1;
}

size_t conv_lds_bytes(const salt_layer_desc* d, const salt_qparams* p, const ConvPlan& pl,
                      bool ext) {
  const int pws = pl.Rw * pl.Wp;
  const ConvLds l = conv_lds_layout(p->n_table, pl.spw, pl.ncg, pl.nsb, pl.nit * pl.Gi, pl.nit,
                                    pl.VS, pl.QS, pws,
                                    conv_pos_words(pws, pl.NC2, conv_spare_pad(pl.Rw, pl.NC)),
                                    ext,
                                    p->v_th_kind == SALT_VTH_PER_NEURON, pl.tsplit != 0,
                                    pl.pair != 0);
  return (size_t)l.words * 4;
}

// The smallest row stride: bands of NC rows or more keep their spare positions in NC
// padding columns.
int min_row_stride(const ConvPlan* pl) {
  return pl->W + (conv_spare_pad(pl->Rw, pl->NC) ? pl->NC : 0);
}

// The plain layout: the smallest row stride, the smallest odd slot strides.
void default_layout(const salt_layer_desc* d, ConvPlan* pl) {
  pl->Wp = min_row_stride(pl);
  pl->VS = conv_pos_words(pl->Rw * pl->Wp, pl->NC2, conv_spare_pad(pl->Rw, pl->NC)) | 1;
  pl->QS = (d->ic * d->k * d->k + 1) | 1;
}

// Cycles one wave64 LDS access takes, as measured on gfx950: the two half-waves are
// served one after the other, each by 32 banks (4-byte words for 32-bit accesses, 8-byte
// words for 64-bit ones), and a half-wave takes as many cycles as the most distinct
// addresses one bank holds (lanes on one address share it).  addr: word addresses,
// -1 = lane without an access; unit: words per bank word (1 or 2).
int lds_access_cycles(const int* addr, int unit) {
  int total = 0;
  for (int h = 0; h < kWave; h += 32) {
    int seen[32][32], cnt[32] = {0}, worst = 0;
    for (int l = h; l < h + 32; ++l) {
      if (addr[l] < 0) continue;
      const int u = addr[l] / unit, bank = u & 31;
      bool dup = false;
      for (int k = 0; k < cnt[bank] && !dup; ++k) dup = seen[bank][k] == u;
      if (!dup) {
        seen[bank][cnt[bank]++] = u;
        worst = std::max(worst, cnt[bank]);
      }
    }
    total += worst;
  }
  return total;
}

// Per-event LDS cycles of a wave's register, weight-code and (time, count) accesses,
// averaged over the 32 bank alignments an event's base can take.  Lane l is slot l / NC2
// (< Gi), candidate (dy, dx) = divmod(l % NC2, NC).
enum ConvAccess { kAccV, kAccQ, kAccTC };
double conv_access_cycles(ConvAccess which, int Gi, int NC, int S, int K, int Wp, int stride) {
  const int NC2 = NC * NC;
  int addr[kWave];
  long sum = 0;
  for (int base = 64; base < 96; ++base) {
    for (int l = 0; l < kWave; ++l) {
      const int slot = l / NC2, cand = l - slot * NC2, dy = cand / NC, dx = cand - dy * NC;
      if (slot >= Gi) { addr[l] = -1; continue; }
      switch (which) {
        case kAccV: addr[l] = 4 * base + slot * stride + dy * Wp + dx; break;
        case kAccQ: addr[l] = 4 * base + slot * stride - dy * S * K - dx * S; break;
        default: addr[l] = 2 * (base + dy * Wp + dx); break;
      }
    }
    sum += lds_access_cycles(addr, which == kAccTC ? 2 : 1);
  }
  return sum / 32.0;
}

// Chooses the row stride Wp >= min_row_stride() and the slot strides VS, QS of a plan
// that minimise the modelled bank-conflict cycles of the event loop's LDS accesses
// (register read + write,
// code read, (time, count) read + write; weights from the measured per-access costs),
// within `budget` bytes of LDS per work-group.  Plans repeat for every call, so the
// choice is cached.
void choose_layout(const salt_layer_desc* d, const salt_qparams* p, bool ext, size_t budget,
                   ConvPlan* pl) {
  default_layout(d, pl);
  const std::array<int, 18> key = {pl->W, pl->Rw, pl->Gi, pl->NC, d->s, d->k, d->ic, pl->nit,
                                   pl->ncg, pl->nsb, pl->spw, p->n_table, (int)ext,
                                   p->v_th_kind == SALT_VTH_PER_NEURON, pl->tsplit, pl->pair,
                                   (int)(budget >> 4), (int)(budget & 15)};
  static std::mutex mu;
  static std::map<std::array<int, 18>, std::array<int, 3>> cache;
  {
    std::lock_guard<std::mutex> g(mu);
    auto it = cache.find(key);
    if (it != cache.end()) {
      pl->Wp = it->second[0]; pl->VS = it->second[1]; pl->QS = it->second[2];
      pl->lds = conv_lds_bytes(d, p, *pl, ext);
      return;
    }
  }
  const int ICKK = d->ic * d->k * d->k;
  int best_qs = pl->QS;
  double best_q = 1e30;
  for (int qs = ICKK + 1; qs < ICKK + 1 + 64; ++qs) {
    const double c = conv_access_cycles(kAccQ, pl->Gi, pl->NC, d->s, d->k, 0, qs);
    if (c < best_q) { best_q = c; best_qs = qs; }
  }
  ConvPlan best = *pl;
  double best_cost = 1e30;
  const int wp0 = min_row_stride(pl);
  for (int wp = wp0; wp <= wp0 + 12; ++wp) {
    const int v0 = conv_pos_words(pl->Rw * wp, pl->NC2, conv_spare_pad(pl->Rw, pl->NC));
    int vs_best = 0;
    double v_best = 1e30;
    for (int vs = v0; vs < v0 + 64; ++vs) {
      const double c = conv_access_cycles(kAccV, pl->Gi, pl->NC, d->s, d->k, wp, vs);
      if (c < v_best) { v_best = c; vs_best = vs; }
    }
    ConvPlan t = *pl;
    t.Wp = wp; t.VS = vs_best; t.QS = best_qs;
    t.lds = conv_lds_bytes(d, p, t, ext);
    if (t.lds > budget) continue;
    const double tc = conv_access_cycles(kAccTC, pl->Gi, pl->NC, d->s, d->k, wp, 0);
    const double cost = 3.2 * v_best + 4.3 * tc + 1.1 * best_q;
    if (cost < best_cost - 1e-9) { best_cost = cost; best = t; }
  }
  if (best_cost < 1e29) *pl = best;
  pl->lds = conv_lds_bytes(d, p, *pl, ext);
  std::lock_guard<std::mutex> g(mu);
  cache[key] = {pl->Wp, pl->VS, pl->QS};
}

// Fills the channel split of a plan: ncg channel groups of G channels, nit iterations
// of Gi slots per event, the fewest iterations whose group count fits max_cg.
bool split_channels(int OC, int max_cg, ConvPlan* pl) {
  for (int nit = 1; nit <= 8; nit = nit < 4 ? nit + 1 : 8 + (nit == 8)) {
    const int ncg = (OC + nit * pl->Gi - 1) / (nit * pl->Gi);
    if (ncg > max_cg) continue;
    pl->ncg = ncg;
    pl->G = (OC + ncg - 1) / ncg;                       // balanced groups
    pl->nit = round_nit((pl->G + pl->Gi - 1) / pl->Gi);
    pl->Gi = (pl->G + pl->nit - 1) / pl->nit;           // no more slots than channels
    return true;
  }
  return false;
}

// Optional override for tuning runs: SALT_CONV_PLAN="ncg_max,nsb" (channel-group limit,
// sub-bands per work-group).  Unset in normal use.
bool plan_override(int* ncg_max, int* nsb) {
  const char* e = getenv("SALT_CONV_PLAN");
  return e && sscanf(e, "%d,%d", ncg_max, nsb) == 2 && *ncg_max >= 1 && *nsb >= 1;
}

// LDS per row-band work-group: kLdsBandBudget, or SALT_CONV_BAND_KB=n KiB (tuning runs).
size_t band_budget() {
  const char* e = getenv("SALT_CONV_BAND_KB");
  const int kb = e ? atoi(e) : 0;
  return kb > 0 ? std::min<size_t>((size_t)kb << 10, kLdsMax) : (size_t)kLdsBandBudget;
}

// SALT_CONV_PAIR=0 / =1 forces steps of one / two events (where candidates fit half a
// wave) for comparisons and tests; both give the same results.  -1: not forced.
int pair_override() {
  const char* e = getenv("SALT_CONV_PAIR");
  if (!e || (e[0] != '0' && e[0] != '1')) return -1;
  return e[0] - '0';
}

// Compute units of the current device (256 on MI355X, the fallback).
int device_cus() {
  static std::mutex mu;
  static std::map<int, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> g(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      n < 1)
    n = 256;
  cache[dev] = n;
  return n;
}

int32_t plan_conv_mode(const salt_layer_desc* d, const salt_qparams* p, int B, bool ext,
                       bool notrunc, bool pair, ConvPlan* pl);

// Chooses between steps of one event and steps of two (a half-wave each, for events
// whose candidate blocks are disjoint; candidates must fit 32 lanes).  Pairs shorten a
// stream's chain of steps -- a lone conv1 stream of configuration 3 0.38 -> 0.32 ms --
// but, with more waves per stream, do more work per event (the steps with one event
// leave half a wave idle), so they pay only while the chip has room for those waves.
// Measured on MI355X (configuration 3, its first B streams, one-event / two-event
// steps): conv1 at B = 256 0.47 / 0.42 ms, at 384 0.50 / 0.57; conv2 (five waves per
// two-event stream against seven for conv1) at 384 0.49 / 0.43, at 512 0.52 / 0.52;
// configuration 2 (nine waves per two-event stream, B = 256) 0.67 / 0.69.  The rule
// that fits them: two-event steps while their plan puts at most kPairWavesPerCu waves on
// a compute unit.
constexpr long kPairWavesPerCu = 8;
int32_t plan_conv(const salt_layer_desc* d, const salt_qparams* p, int B, bool ext,
                  bool notrunc, ConvPlan* pl) {
  const int NC = (d->k - 1) / std::max(d->s, 1) + 1;
  const int force = pair_override();
  if (NC * NC <= kWave / 2 && force != 0) {
    const int32_t rc = plan_conv_mode(d, p, B, ext, notrunc, true, pl);
    if (rc) return rc;
    const long waves = (long)B * pl->n_rb * conv_block_waves(pl->spw, pl->ncg, pl->nsb);
    if (force == 1 || waves <= kPairWavesPerCu * device_cus()) return 0;
  }
  return plan_conv_mode(d, p, B, ext, notrunc, false, pl);
}

// Chooses the partition of a conv layer.  One work-group per stream holds the whole
// output plane whenever its LDS fits; its waves are channel groups, each with one
// iteration per event where 8 waves suffice (a lone wave per SIMD is latency-bound,
// and channel groups see the same events, so they stay in step between the per-chunk
// barriers; row sub-bands are supported but unbalanced for clustered events).
// Otherwise several work-groups per stream each take a band of rows.
// notrunc: max_queue_len >= the stream length, so no queue can be truncated.
// pair: steps of two events (needs NC2 <= 32).
int32_t plan_conv_mode(const salt_layer_desc* d, const salt_qparams* p, int B, bool ext,
                       bool notrunc, bool pair, ConvPlan* pl) {
  pl->tsplit = notrunc ? 1 : 0;
  pl->H = (d->h_in + 2 * d->p - d->k) / d->s + 1;
  pl->W = (d->w_in + 2 * d->p - d->k) / d->s + 1;
  if (pl->H < 1 || pl->W < 1) return fail(-1, "conv geometry gives an empty output plane");
  pl->HW = pl->H * pl->W;
  pl->NC = (d->k - 1) / d->s + 1;
  pl->NC2 = pl->NC * pl->NC;
  if (pl->NC2 > kWave)
    return fail(-3, "conv: %d candidate positions per event (k=%d, s=%d) exceed 64", pl->NC2,
                d->k, d->s);
  pl->pair = pair && pl->NC2 <= kWave / 2 ? 1 : 0;
  pl->Gi = (pl->pair ? kWave / 2 : kWave) / pl->NC2;  // slots per (half-)wave
  const int H = pl->H, OC = d->oc;
  int ncg_max = kConvMaxWaves, nsb = 1;
  plan_override(&ncg_max, &nsb);
  if (!split_channels(OC, ncg_max, pl) && !split_channels(OC, kConvMaxWaves, pl))
    return fail(-3, "conv: %d output channels need more than 8 iterations", OC);
  nsb = std::max(1, std::min(nsb, kConvMaxWaves / pl->ncg));
  pl->Rw = (H + nsb - 1) / nsb;
  pl->nsb = (H + pl->Rw - 1) / pl->Rw;                // no empty sub-band
  pl->R = H; pl->n_rb = 1; pl->merge = 1; pl->spw = 1;
  default_layout(d, pl);
  pl->lds = conv_lds_bytes(d, p, *pl, ext);
  if (pl->lds <= (size_t)kLdsMax) {
    // padding may not cost a work-group per compute unit
    const size_t per_cu = std::max<size_t>(1, (size_t)kLdsMax / pl->lds);
    choose_layout(d, p, ext, (size_t)kLdsMax / per_cu, pl);
    return 0;
  }
  // Bands of rows, one work-group (of channel-group waves) each, within the budget.
  pl->nsb = 1; pl->merge = 0;
  const size_t budget = band_budget();
  int R = H;
  for (;;) {
    pl->Rw = pl->R = R;
    default_layout(d, pl);
    pl->lds = conv_lds_bytes(d, p, *pl, ext);
    if (pl->lds <= budget || R == 1) break;
    --R;
  }
  if (pl->lds > (size_t)kLdsMax)
    return fail(-3, "conv: one output row does not fit in LDS (w_out=%d)", pl->W);
  pl->n_rb = (H + R - 1) / R;
  choose_layout(d, p, ext, std::max(pl->lds, budget), pl);
  return 0;
}

// Whole-plane plans: whether the helper wave places every channel group's spikes (the
// channel groups then run nothing but their events), or each channel-group wave its own.
// One helper keeps up with up to kConvHelperWalks (channel group, iteration) pairs: on
// configuration 3 (3 and 2 of them) it takes conv1 0.73 -> 0.69 ms and conv2 0.64 ->
// 0.54 ms, on configuration 2 with steps of one event (8) 0.666 -> 0.659 ms; with 16
// (configuration 2 with steps of two events: 8 groups of two iterations) it takes twice
// as long per chunk as the channel groups (0.71 -> 0.78 ms).  SALT_CONV_HWALK=0 / =1
// forces either for comparisons and tests; both give the same results.
constexpr int kConvHelperWalks = 8;
int helper_walks(const ConvPlan& pl) {
  const char* e = getenv("SALT_CONV_HWALK");
  if (e && (e[0] == '0' || e[0] == '1')) return e[0] - '0';
  return pl.ncg * pl.nit <= kConvHelperWalks ? 1 : 0;
}

// Issue priority of the helper waves: 1 where their per-chunk work is heavy -- placing
// the spikes of kConvHelperPrioWalks or more (channel group, iteration) pairs, or storing
// a row band's spike words -- else 0, below the channel-group waves for most of each
// chunk.  Measured on MI355X (priority 0 / 1): configuration 2 (8 pairs) 0.660-0.663 /
// 0.624-0.637 ms, configuration 4 (row bands) 2.257 / 2.242-2.250 ms; configuration 3's
// conv2 (2 pairs) 0.546-0.548 / 0.550-0.552 ms, conv1 (3 pairs) unchanged.  Steps of two
// events keep 0 (not measured there).
constexpr int kConvHelperPrioWalks = 4;
int helper_priority(const ConvPlan& pl, int hwalk) {
  if (pl.pair) return 0;
  if (!pl.merge) return 1;
  return hwalk && pl.ncg * pl.nit >= kConvHelperPrioWalks ? 1 : 0;
}

// Streams per work-group of a whole-plane plan: one unless SALT_CONV_SPW=n asks for n
// (within 16 waves and the LDS).  Several streams per work-group advance chunk by chunk
// together, behind one barrier; on configuration 3 that was slower than independent
// work-groups (the waves that finish a chunk first wait for the others), so it is a
// tuning option, covered by the parity tests.
void choose_spw(const salt_layer_desc* d, const salt_qparams* p, int B, bool ext,
                ConvPlan* pl) {
  if (!pl->merge) return;
  const int nwps = pl->ncg * pl->nsb + pl->nsb;  // with the helper waves
  const char* e = getenv("SALT_CONV_SPW");
  int spw = e ? atoi(e) : 1;
  if (spw <= 1) return;
  spw = std::min({spw, kConvBlockWaves / nwps, std::max(B, 1)});
  for (; spw > 1; --spw) {
    ConvPlan t = *pl;
    t.spw = spw;
    const size_t lds = conv_lds_bytes(d, p, t, ext);
    if (lds <= (size_t)kLdsMax) {
      pl->spw = spw;
      pl->lds = lds;
      return;
    }
  }
}

// ------------------------------------------------------------------ packed conv plan

struct PackPlan {
  int H, W, NC, ncg, Gw, spw, P, imax, Wp, VS, QS;
  bool vtha;
  size_t lds;
};

// The packed conv kernel runs only when asked for: SALT_CONV_PACKED=1, or
// SALT_CONV_PACK="ncg,spw" (which also forces its channel groups and streams per
// work-group).  Measured on MI355X it is slower than the channel-slot kernel on every
// configuration (configuration 3 at B=1024: conv1 1.04 ms against 0.75, conv2 0.67
// against 0.65; configuration 2: 0.95 against 0.69), so the channel-slot kernel is the
// default.  Results never depend on the choice.
bool packed_disabled() {
  const char* e = getenv("SALT_CONV_PACKED");
  if (e) return e[0] != '1';
  return getenv("SALT_CONV_PACK") == nullptr;
}
bool pack_override(int* ncg, int* spw) {
  const char* e = getenv("SALT_CONV_PACK");
  return e && sscanf(e, "%d,%d", ncg, spw) == 2 && *ncg >= 1 && *spw >= 1;
}

size_t pack_lds_bytes(const salt_qparams* p, const PackPlan& pl, bool ext, bool notrunc) {
  const PackLds l = pack_lds_layout(p->n_table, pl.NC * pl.NC, pl.ncg, pl.spw, pl.P, pl.VS, pl.QS,
                                    pl.H * pl.Wp, pl.imax, ext, pl.vtha, notrunc);
  return (size_t)l.words * 4;
}

// Plans the packed kernel for a conv layer whose output plane (all channels, with the
// zero planes) fits in LDS with candidate grids of at most kPackMaxNC^2 positions.
// Channel groups (waves per stream): enough for one wave per SIMD over the batch (a
// stream's single wave when the batch fills the chip), each group at most 8 iterations
// per event; streams per work-group: up to 4 independent single-wave streams sharing
// the tables and codes.  Returns false when the layer does not qualify.
bool plan_packed(const salt_layer_desc* d, const salt_qparams* p, int B, bool ext, bool notrunc,
                 PackPlan* pl) {
  if (packed_disabled()) return false;
  pl->H = (d->h_in + 2 * d->p - d->k) / d->s + 1;
  pl->W = (d->w_in + 2 * d->p - d->k) / d->s + 1;
  if (pl->H < 1 || pl->W < 1) return false;
  pl->NC = (d->k - 1) / d->s + 1;
  if (pl->NC > kPackMaxNC) return false;
  pl->vtha = p->v_th_kind == SALT_VTH_PER_CHANNEL || p->v_th_kind == SALT_VTH_PER_NEURON;
  const int OC = d->oc, cus = device_cus();
  const int max_g = std::min(kPackMaxBlockWaves, OC);
  int ncg = std::max(1, std::min(max_g, (4 * cus + std::max(B, 1) - 1) / std::max(B, 1)));
  int spw = 0;
  const bool forced = pack_override(&ncg, &spw);
  ncg = std::min(ncg, max_g);
  for (;; ++ncg) {
    if (ncg > max_g) return false;
    pl->ncg = ncg;
    pl->Gw = (OC + ncg - 1) / ncg;
    int imax = 0;
    pl->P = pack_slots(pl->NC, pl->Gw, &imax);
    if (imax <= 8) { pl->imax = imax; break; }
  }
  pl->Wp = pl->W;
  pl->VS = pl->H * pl->W;
  pl->QS = d->ic * d->k * d->k;
  // streams per work-group: up to 4 (with one wave each) or 2 (with several), within the
  // work-group size
  const int spw_cap = kPackMaxBlockWaves / pl->ncg;
  const int spw_max = std::min(spw_cap, forced ? spw : (pl->ncg == 1 ? 4 : 2));
  for (pl->spw = std::max(1, std::min(spw_max, std::max(B, 1))); pl->spw >= 1; --pl->spw) {
    pl->lds = pack_lds_bytes(p, *pl, ext, notrunc);
    if (pl->lds <= (size_t)kLdsMax) return true;
  }
  return false;
}

struct FcPlan {
  int npl, n_slices, words, direct, wpg;
};

// Waves per stream of a directly appending FC layer: SALT_FC_WAVES=n (1..kFcMaxWaves)
// for tuning runs and tests, else 4.  Measured on MI355X: configuration 1 (128 neurons,
// one stream) 0.42 -> 0.30 ms with two waves of 64 instead of one of 128; configuration 5
// (1024 neurons, 4096 streams, ~180 spikes per event, dense chunks placed with one run
// of entries per store) 31.0-32.4 ms with two waves of 512, 24.0-25.1 ms with four of
// 256, 29.8-30.7 ms with eight of 128 (a build allowing eight).
int fc_waves_limit() {
  const char* e = getenv("SALT_FC_WAVES");
  const int n = e ? atoi(e) : 4;
  return std::max(1, std::min(n, kFcMaxWaves));
}

// One stream's neurons go to wpg waves of 64*npl neurons (npl a power of two <= 16).
// Up to kFcMaxWaves x 1024 neurons the waves form one work-group that appends to the
// stream directly; beyond, each slice of 1024 is a work-group writing spike masks.
// Several waves of fewer neurons each, rather than one wave of many: a wave of 1024
// neurons needs over 256 registers (one wave per SIMD, nothing hides its memory
// waits), and each wave's chain of events is shorter.
int32_t plan_fc(const salt_layer_desc* d, FcPlan* pl) {
  const int need = (d->n_out + kWave - 1) / kWave;  // 64-neuron words
  const int wmax = fc_waves_limit();
  int npl = 1;
  if (need <= 16 * wmax) {
    while (npl * wmax < need) npl *= 2;
    pl->wpg = (need + npl - 1) / npl;               // no wave without a neuron
    pl->n_slices = 1;
  } else {
    npl = 16;
    pl->wpg = 1;
    pl->n_slices = (need + npl - 1) / npl;
  }
  pl->npl = npl;
  pl->words = (d->n_out + 31) / 32;
  pl->direct = pl->n_slices == 1;
  return 0;
}

int32_t check_common(const salt_layer_desc* d, const salt_qparams* p) {
  if (!d || !p) return fail(-1, "null descriptor");
  if (p->f_a < 0 || p->f_a > 15)
    return fail(-1, "shift_bits=%d above MAX_SHIFT_BITS=15 (or negative)", p->f_a);
  if (p->f_V < 0) return fail(-1, "f_V=%d is negative", p->f_V);
  if (p->i_V + p->f_V > 30)
    return fail(-1, "total_bits=%d above MAX_REGISTER_BITS=30", p->i_V + p->f_V);
  if (p->i_V + p->f_V < 1) return fail(-1, "total_bits=%d below 1", p->i_V + p->f_V);
  if (p->n_table < 1) return fail(-1, "decay table is empty");
  if (p->n_table > kMaxTable) return fail(-1, "decay table longer than %d entries", kMaxTable);
  if (p->q_bits != 8 && p->q_bits != 16 && p->q_bits != 32)
    return fail(-1, "q_bits must be 8, 16 or 32, got %d", p->q_bits);
  if (p->round_mode != SALT_ROUND && p->round_mode != SALT_TRUNCATE)
    return fail(-1, "invalid round_mode %d", p->round_mode);
  if (p->overflow_mode != SALT_WRAP && p->overflow_mode != SALT_SATURATE)
    return fail(-1, "invalid overflow_mode %d", p->overflow_mode);
  if (p->v_th_kind < SALT_VTH_NONE || p->v_th_kind > SALT_VTH_PER_NEURON)
    return fail(-1, "invalid v_th_kind %d", p->v_th_kind);
  if (p->v_th_kind == SALT_VTH_SCALAR && p->v_th_scalar <= 0)
    return fail(-1, "v_th_int must be > 0, got %d", p->v_th_scalar);
  if ((p->v_th_kind == SALT_VTH_PER_CHANNEL || p->v_th_kind == SALT_VTH_PER_NEURON) &&
      !p->d_v_th)
    return fail(-1, "v_th array missing");
  if (!p->d_q || !p->d_decay_table) return fail(-1, "weights or decay table missing");
  if (d->max_out_spikes < 0) return fail(-1, "max_out_spikes < 0");
  if (d->kind == SALT_LAYER_FC) {
    if (d->n_in < 1 || d->n_out < 1) return fail(-1, "FC needs n_in, n_out >= 1");
    if (p->v_th_kind == SALT_VTH_PER_NEURON) return fail(-1, "FC: use SALT_VTH_PER_CHANNEL");
  } else if (d->kind == SALT_LAYER_CONV) {
    if (d->ic < 1 || d->h_in < 1 || d->w_in < 1 || d->oc < 1 || d->k < 1 || d->s < 1 ||
        d->p < 0)
      return fail(-1, "invalid conv geometry");
    if (d->max_queue_len < 1) return fail(-1, "max_queue_len must be >= 1");
  } else {
    return fail(-1, "unknown layer kind %d", d->kind);
  }
  return 0;
}

Quant make_quant(const salt_qparams* p) {
  Quant q;
  q.fa = p->f_a;
  q.fV = p->f_V;
  q.wbits = p->i_V + p->f_V;
  q.rc = (p->round_mode == SALT_ROUND && p->f_a > 0) ? (1 << (p->f_a - 1)) : 0;
  q.half = 1 << (q.wbits - 1);
  q.n_table = p->n_table;
  q.vth_kind = p->v_th_kind;
  q.vth_scalar = p->v_th_scalar;
  q.vth = p->d_v_th;
  return q;
}

ConvGeom conv_geom(const salt_layer_desc* d, const ConvPlan& pl) {
  ConvGeom g;
  g.IC = d->ic; g.Win = d->w_in; g.HWin = d->h_in * d->w_in; g.OC = d->oc;
  g.K = d->k; g.S = d->s; g.P = d->p; g.H = pl.H; g.W = pl.W; g.HW = pl.HW;
  g.NC = pl.NC; g.NC2 = pl.NC2; g.mql = d->max_queue_len;
  g.Wp = pl.Wp;
  g.rHWin = 1.0f / (float)g.HWin;  // correctly rounded on the host
  g.rWin = 1.0f / (float)g.Win;
  g.rS = 1.0f / (float)g.S;
  return g;
}

// Workspace of a compacted layer: the spikes (FC slices: bit masks; conv row bands: the
// validity words, then the spike words), then (256-byte aligned) the spikes per (stream,
// segment) of the compaction.
size_t masks_end(size_t mask_bytes) { return (mask_bytes + 255) & ~(size_t)255; }
size_t compact_bytes(size_t mask_bytes, int B, int L) {
  return masks_end(mask_bytes) + (size_t)B * compact_segments(L) * 4;
}
// Bands an event reaches at most: its NC candidate rows meet ceil((NC-1)/R) + 1 bands.
int band_slots(const ConvPlan& pl) { return (pl.NC - 1 + pl.R - 1) / pl.R + 1; }
size_t valid_bytes_conv(int B, int L) { return masks_end((size_t)B * L * 4); }
size_t spike_bytes_conv(const ConvPlan& pl, int B, int L) {
  return valid_bytes_conv(B, L) + (size_t)B * L * band_slots(pl) * pl.ncg * pl.nit * 8;
}
// Row-band event lists (band_count/scan/fill_kernel): entries per stream, one per band an
// event reaches; 0 when lists are off (SALT_CONV_BANDLIST=0, for comparisons), the bands
// exceed the list build's LDS or the entries would not fit 32-bit indices.
long band_cap(const ConvPlan& pl, int L) {
  const char* e = getenv("SALT_CONV_BANDLIST");
  if (pl.merge || pl.n_rb > kBandMaxRb || (e && e[0] == '0')) return 0;
  const long cap = (long)L * band_slots(pl);
  return cap <= INT_MAX ? cap : 0;
}
int band_segments(int L) { return std::max(1, (L + kBandSeg - 1) / kBandSeg); }
// lengths and offsets, the lists, the per-segment places
size_t band_bytes(const ConvPlan& pl, int B, int L) {
  const long cap = band_cap(pl, L);
  return cap ? (size_t)B * pl.n_rb * 2 * 4 + (size_t)B * cap * 4 +
                   (size_t)B * band_segments(L) * pl.n_rb * 4
             : 0;
}
size_t mask_bytes_conv(const ConvPlan& pl, int B, int L) {
  if (pl.merge) return 0;
  return masks_end(compact_bytes(spike_bytes_conv(pl, B, L), B, L)) + band_bytes(pl, B, L);
}
size_t mask_only_fc(const FcPlan& pl, int B, int L) { return (size_t)B * L * pl.words * 4; }
size_t mask_bytes_fc(const FcPlan& pl, int B, int L) {
  return pl.direct ? 0 : compact_bytes(mask_only_fc(pl, B, L), B, L);
}

int32_t* compact_seg_counts(void* ws, size_t mask_bytes) {
  return reinterpret_cast<int32_t*>(static_cast<char*>(ws) + masks_end(mask_bytes));
}

// Launches the two compaction kernels over an FC layer's spike masks.
int32_t launch_compact(const CompactArgs& c, int B, int L, size_t mask_bytes, void* ws,
                       hipStream_t st) {
  const int nseg = compact_segments(L);
  int32_t* const seg = compact_seg_counts(ws, mask_bytes);
  const dim3 grid(nseg, B);
  hipLaunchKernelGGL(compact_count_kernel, grid, dim3(kWave), 0, st, c, seg, nseg);
  HIP_TRY(hipGetLastError());
  hipLaunchKernelGGL(compact_kernel, grid, dim3(kWave), 0, st, c, (const int32_t*)seg, nseg);
  HIP_TRY(hipGetLastError());
  return 0;
}

int32_t fill(int32_t* p, int32_t v, size_t n, hipStream_t st) {
  if (n == 0) return 0;
  const size_t blocks = std::min<size_t>((n + 255) / 256, 65536);
  hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)blocks), dim3(256), 0, st, p, v, n);
  HIP_TRY(hipGetLastError());
  return 0;
}

hipError_t launch_conv(const ConvArgs& a, const ConvPlan& pl, int flags, int B,
                       hipStream_t st) {
  const dim3 grid(pl.n_rb, (B + pl.spw - 1) / pl.spw),
      block(kWave * conv_block_waves(pl.spw, pl.ncg, pl.nsb));
  switch (pl.nit) {
#define SALT_CASE(N) \
    case N: return launch_conv_nit##N(a, flags, grid, block, pl.lds, st);
    SALT_CONV_NITS(SALT_CASE)
#undef SALT_CASE
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_pack(const PackArgs& a, const PackPlan& pl, int flags, dim3 grid,
                       hipStream_t st) {
  const dim3 block(kWave * pl.ncg * pl.spw);
  switch (pl.imax) {
#define SALT_CASE(N) \
    case N: return launch_pack_imax##N(a, flags, grid, block, pl.lds, st);
    SALT_PACK_IMAXES(SALT_CASE)
#undef SALT_CASE
    default: return hipErrorInvalidValue;
  }
}

// Enqueues one conv layer on the packed kernel (arguments already checked).
int32_t launch_packed(const salt_layer_desc* desc, const salt_qparams* prm,
                      const salt_events_in* in, const salt_events_out* out,
                      const salt_layer_result* res, const Quant& qz, const PackPlan& pl, int B,
                      int L, bool ext, bool sat, bool notrunc, hipStream_t st) {
  PackArgs a;
  a.g.IC = desc->ic; a.g.Win = desc->w_in; a.g.HWin = desc->h_in * desc->w_in; a.g.OC = desc->oc;
  a.g.K = desc->k; a.g.S = desc->s; a.g.P = desc->p; a.g.H = pl.H; a.g.W = pl.W;
  a.g.HW = pl.H * pl.W; a.g.NC = pl.NC; a.g.NC2 = pl.NC * pl.NC; a.g.mql = desc->max_queue_len;
  a.g.Wp = pl.Wp;
  a.g.rHWin = 1.0f / (float)a.g.HWin;  // correctly rounded on the host
  a.g.rWin = 1.0f / (float)a.g.Win;
  a.g.rS = 1.0f / (float)a.g.S;
  a.ncls = pl.NC * pl.NC;
  a.ncg = pl.ncg; a.Gw = pl.Gw; a.spw = pl.spw; a.B = B;
  a.P = pl.P; a.VS = pl.VS; a.QS = pl.QS;
  a.qz = qz; a.table = prm->d_decay_table; a.q = prm->d_q; a.q_bits = prm->q_bits;
  a.L = L; a.times = in->d_times; a.src = in->d_src; a.n_real = in->d_n_real;
  a.cap = out->cap; a.fill_pads = out->fill_pads;
  a.out_t = out->d_times; a.out_s = out->d_src; a.out_n = out->d_n;
  a.v_final = res->d_v_final; a.v_min = res->d_v_min; a.v_max = res->d_v_max;
  a.stats = res->d_stats;
  const int flags = (sat ? kPackSat : 0) | (ext ? kPackExt : 0) | (pl.vtha ? kPackVtha : 0) |
                    (notrunc ? kPackNoTrunc : 0);
  const dim3 grid((B + pl.spw - 1) / pl.spw);
  HIP_TRY(launch_pack(a, pl, flags, grid, st));
  return 0;
}

constexpr size_t kFcWeightLds = 40 * 1024;  // stage FC weight slices up to this size

// Checks the arguments of one layer call (launch = 0) or, once they are known to be
// valid, enqueues it on st (launch = 1).
int32_t layer_forward(const salt_layer_desc* desc, const salt_qparams* prm,
                      const salt_events_in* in, const salt_events_out* out,
                      const salt_layer_result* res, void* d_workspace, size_t workspace_bytes,
                      hipStream_t st, int launch) {
  int32_t rc = check_common(desc, prm);
  if (rc) return rc;
  if (!in || !out || !res) return fail(-1, "null events or result descriptor");
  const int B = in->B, L = in->L;
  if (B < 0 || L < 0) return fail(-1, "invalid batch shape B=%d L=%d", B, L);
  if (B > 65535) return fail(-1, "batch of %d streams above 65535", B);
  if (B == 0) return 0;
  if (!in->d_n_real || (L > 0 && (!in->d_times || !in->d_src)))
    return fail(-1, "input events missing");
  if (out->cap != desc->max_out_spikes) return fail(-1, "out.cap must equal max_out_spikes");
  if (!out->d_n || (out->cap > 0 && (!out->d_times || !out->d_src)))
    return fail(-1, "output stream buffers missing");
  if (!res->d_stats) return fail(-1, "stats buffer missing");
  if ((res->d_v_min == nullptr) != (res->d_v_max == nullptr))
    return fail(-1, "give both or neither of v_min/v_max");
  const bool ext = res->d_v_min != nullptr;
  const Quant qz = make_quant(prm);
  const bool sat = prm->overflow_mode == SALT_SATURATE;

  if (desc->kind == SALT_LAYER_CONV) {
    const bool notrunc = desc->max_queue_len >= L;
    PackPlan pk;
    if (plan_packed(desc, prm, B, ext, notrunc, &pk)) {
      if (!launch) return 0;
      return launch_packed(desc, prm, in, out, res, qz, pk, B, L, ext, sat, notrunc, st);
    }
    ConvPlan pl;
    rc = plan_conv(desc, prm, B, ext, notrunc, &pl);
    if (rc) return rc;
    const size_t need = mask_bytes_conv(pl, B, L);
    if (workspace_bytes < need || (need && !d_workspace))
      return fail(-1, "workspace of %zu bytes below the %zu needed", workspace_bytes, need);
    if (!launch) return 0;
    choose_spw(desc, prm, B, ext, &pl);
    ConvArgs a;
    a.seg_cnt = nullptr; a.nseg = 0;  // row bands: set below
    a.g = conv_geom(desc, pl);
    a.G = pl.G; a.Gi = pl.Gi; a.ncg = pl.ncg; a.nsb = pl.nsb; a.Rw = pl.Rw; a.R = pl.R;
    a.spw = pl.spw; a.B = B;
    a.VS = pl.VS; a.QS = pl.QS;
    a.qz = qz; a.table = prm->d_decay_table; a.q = prm->d_q; a.q_bits = prm->q_bits;
    a.L = L; a.times = in->d_times; a.src = in->d_src; a.n_real = in->d_n_real;
    a.cap = out->cap; a.fill_pads = out->fill_pads; a.merge = pl.merge;
    a.hwalk = helper_walks(pl);
    a.hprio = helper_priority(pl, a.hwalk);
    a.out_t = out->d_times; a.out_s = out->d_src; a.out_n = out->d_n;
    a.v_final = res->d_v_final; a.v_min = res->d_v_min; a.v_max = res->d_v_max;
    a.stats = res->d_stats;
    // row bands: validity words, spike words, segment counts, event lists
    a.valid = static_cast<uint32_t*>(d_workspace);
    a.words = reinterpret_cast<uint64_t*>(static_cast<char*>(d_workspace) +
                                          valid_bytes_conv(B, L));
    a.nslots = pl.merge ? 0 : band_slots(pl);
    a.blist = nullptr; a.bcnt = nullptr; a.boff = nullptr; a.bcap = 0;
    if (const long cap = band_cap(pl, L)) {  // row bands: each band's events, listed
      BandArgs ba;
      ba.L = L; ba.R = pl.R; ba.H = pl.H; ba.n_rb = pl.n_rb; ba.K = desc->k; ba.S = desc->s;
      ba.P = desc->p; ba.HWin = a.g.HWin; ba.Win = desc->w_in; ba.n_src = desc->ic * a.g.HWin;
      ba.cap = (int)cap; ba.nseg = band_segments(L);
      ba.rHWin = a.g.rHWin; ba.rWin = a.g.rWin; ba.rS = a.g.rS; ba.rR = 1.0f / (float)pl.R;
      ba.src = in->d_src; ba.n_real = in->d_n_real;
      ba.cnt = reinterpret_cast<int32_t*>(
          static_cast<char*>(d_workspace) +
          masks_end(compact_bytes(spike_bytes_conv(pl, B, L), B, L)));
      ba.off = ba.cnt + (size_t)B * pl.n_rb;
      ba.list = ba.off + (size_t)B * pl.n_rb;
      ba.seg_pos = ba.list + (size_t)B * cap;
      const dim3 sgrid(ba.nseg, B);
      hipLaunchKernelGGL(band_count_kernel, sgrid, dim3(kWave), 0, st, ba);
      HIP_TRY(hipGetLastError());
      hipLaunchKernelGGL(band_scan_kernel, dim3(B), dim3(kWave), 0, st, ba);
      HIP_TRY(hipGetLastError());
      hipLaunchKernelGGL(band_fill_kernel, sgrid, dim3(kWave), (size_t)pl.n_rb * 12, st, ba,
                         band_slots(pl));
      HIP_TRY(hipGetLastError());
      a.blist = ba.list; a.bcnt = ba.cnt; a.boff = ba.off; a.bcap = ba.cap;
    }
    if (!pl.merge) {
      if ((rc = fill(res->d_stats, 0, (size_t)B * 4, st))) return rc;
      if ((rc = fill(reinterpret_cast<int32_t*>(a.valid), 0, (size_t)B * L, st))) return rc;
      a.nseg = compact_segments(L);
      a.seg_cnt = compact_seg_counts(d_workspace, spike_bytes_conv(pl, B, L));
      if ((rc = fill(a.seg_cnt, 0, (size_t)B * a.nseg, st))) return rc;
    }
    const int flags = (sat ? kConvSat : 0) | (ext ? kConvExt : 0) |
                      (prm->v_th_kind == SALT_VTH_PER_NEURON ? kConvVthN : 0) |
                      (pl.NC2 <= 32 ? kConvM32 : 0) |
                      (pl.tsplit ? kConvNoTrunc : 0) |  // the layout follows these two
                      (pl.pair ? kConvPair : 0);
    HIP_TRY(launch_conv(a, pl, flags, B, st));
    if (!pl.merge) {
      BandCompactArgs c;
      c.L = L; c.HW = pl.HW; c.W = pl.W; c.HWin = a.g.HWin; c.Win = desc->w_in; c.K = desc->k;
      c.S = desc->s; c.P = desc->p; c.NC = pl.NC; c.NC2 = pl.NC2; c.OC = desc->oc;
      c.G = pl.G; c.Gi = pl.Gi; c.nit = pl.nit; c.ncg = pl.ncg; c.nslots = a.nslots;
      c.times = in->d_times; c.src = in->d_src; c.n_real = in->d_n_real;
      c.words = a.words; c.valid = a.valid;
      c.cap = out->cap; c.fill_pads = out->fill_pads;
      c.out_t = out->d_times; c.out_s = out->d_src; c.out_n = out->d_n;
      hipLaunchKernelGGL(band_compact_kernel, dim3(a.nseg, B), dim3(kWave), 0, st, c,
                         (const int32_t*)a.seg_cnt, a.nseg);
      HIP_TRY(hipGetLastError());
    }
    return 0;
  }

  FcPlan pl;
  plan_fc(desc, &pl);
  const size_t need = mask_bytes_fc(pl, B, L);
  if (workspace_bytes < need || (need && !d_workspace))
    return fail(-1, "workspace of %zu bytes below the %zu needed", workspace_bytes, need);
  const size_t sw = (size_t)std::min(kWave * pl.npl, desc->n_out);
  const size_t wbytes = (size_t)desc->n_in * sw * (prm->q_bits / 8);
  const size_t tbytes = (size_t)fc_lds_table_words(prm->n_table) * 4;
  // the waves of a multi-wave work-group read weights from global memory (L2)
  const bool wlds = pl.wpg == 1 && wbytes + tbytes <= kFcWeightLds;
  const size_t merge = pl.wpg > 1 ? (size_t)(2 * kFcMaxWaves * kWave + 2 * kFcMaxWaves) * 4 : 0;
  const size_t lds = tbytes + (wlds ? wbytes : 0) + merge;
  if (lds > (size_t)kLdsMax) return fail(-3, "decay table too long for LDS");
  if (!launch) return 0;
  FcArgs a;
  a.n_in = desc->n_in; a.n_out = desc->n_out; a.words = pl.words;
  a.qz = qz; a.table = prm->d_decay_table; a.qt = prm->d_q; a.q_bits = prm->q_bits;
  a.L = L; a.times = in->d_times; a.src = in->d_src; a.n_real = in->d_n_real;
  a.cap = out->cap; a.fill_pads = out->fill_pads; a.direct = pl.direct;
  a.out_t = out->d_times; a.out_s = out->d_src; a.out_n = out->d_n;
  a.v_final = res->d_v_final; a.v_min = res->d_v_min; a.v_max = res->d_v_max;
  a.stats = res->d_stats;
  a.masks = static_cast<uint32_t*>(d_workspace);
  if (!pl.direct && (rc = fill(res->d_stats, 0, (size_t)B * 4, st))) return rc;
  const int flags = (sat ? kFcSat : 0) | (wlds ? kFcWlds : 0) |
                    (prm->v_th_kind == SALT_VTH_NONE ? kFcNoFire : 0);
  const dim3 grid(pl.n_slices, B);
  switch (prm->q_bits) {
    case 8: HIP_TRY(launch_fc_q8(a, pl.npl, flags, grid, pl.wpg, lds, st)); break;
    case 16: HIP_TRY(launch_fc_q16(a, pl.npl, flags, grid, pl.wpg, lds, st)); break;
    default: HIP_TRY(launch_fc_q32(a, pl.npl, flags, grid, pl.wpg, lds, st)); break;
  }
  if (!pl.direct) {
    CompactArgs c;
    memset(&c, 0, sizeof(c));
    c.words = pl.words; c.L = L; c.times = in->d_times;
    c.n_real = in->d_n_real; c.masks = a.masks; c.cap = out->cap;
    c.fill_pads = out->fill_pads; c.out_t = out->d_times; c.out_s = out->d_src;
    c.out_n = out->d_n;
    if ((rc = launch_compact(c, B, L, mask_only_fc(pl, B, L), d_workspace, st))) return rc;
  }
  return 0;
}

}  // namespace

// ------------------------------------------------------------------ C-ABI

extern "C" {

int32_t salt_version(void) { return SALT_ABI_VERSION; }

const char* salt_last_error(void) { return g_err.c_str(); }

int32_t salt_malloc(void** d_ptr, size_t bytes) {
  if (!d_ptr) return fail(-1, "null output pointer");
  HIP_TRY(hipMalloc(d_ptr, bytes));
  return 0;
}

int32_t salt_free(void* d_ptr) {
  HIP_TRY(hipFree(d_ptr));
  return 0;
}

int32_t salt_memcpy_h2d(void* d_dst, const void* h_src, size_t bytes, void* stream) {
  HIP_TRY(hipMemcpyAsync(d_dst, h_src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream));
  return 0;
}

int32_t salt_memcpy_d2h(void* h_dst, const void* d_src, size_t bytes, void* stream) {
  HIP_TRY(hipMemcpyAsync(h_dst, d_src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream));
  return 0;
}

int32_t salt_stream_sync(void* stream) {
  HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
  return 0;
}

int32_t salt_fc_transpose(const void* d_q_ref, void* d_q_t, int32_t n_out, int32_t n_in,
                          int32_t q_bits, void* stream) {
  if (!d_q_ref || !d_q_t || n_out < 1 || n_in < 1) return fail(-1, "invalid transpose args");
  dim3 grid((n_in + 31) / 32, (n_out + 31) / 32), block(32, 8);
  hipStream_t st = (hipStream_t)stream;
  switch (q_bits) {
    case 8:
      hipLaunchKernelGGL(transpose_kernel<int8_t>, grid, block, 0, st,
                         (const int8_t*)d_q_ref, (int8_t*)d_q_t, n_out, n_in);
      break;
    case 16:
      hipLaunchKernelGGL(transpose_kernel<int16_t>, grid, block, 0, st,
                         (const int16_t*)d_q_ref, (int16_t*)d_q_t, n_out, n_in);
      break;
    case 32:
      hipLaunchKernelGGL(transpose_kernel<int32_t>, grid, block, 0, st,
                         (const int32_t*)d_q_ref, (int32_t*)d_q_t, n_out, n_in);
      break;
    default:
      return fail(-1, "q_bits must be 8, 16 or 32");
  }
  HIP_TRY(hipGetLastError());
  return 0;
}

int32_t salt_layer_workspace_size(const salt_layer_desc* desc, const salt_qparams* prm,
                                  int32_t B, int32_t L, int32_t want_neuron_extremes,
                                  size_t* bytes) {
  int32_t rc = check_common(desc, prm);
  if (rc) return rc;
  if (!bytes || B < 0 || L < 0) return fail(-1, "invalid batch shape");
  if (desc->kind == SALT_LAYER_CONV) {
    PackPlan pk;
    if (plan_packed(desc, prm, B, want_neuron_extremes != 0, desc->max_queue_len >= L, &pk)) {
      *bytes = 0;  // the packed kernel keeps everything in LDS
      return 0;
    }
    ConvPlan pl;
    rc = plan_conv(desc, prm, B, want_neuron_extremes != 0, desc->max_queue_len >= L, &pl);
    if (rc) return rc;
    *bytes = mask_bytes_conv(pl, B, L);
  } else {
    FcPlan pl;
    plan_fc(desc, &pl);
    *bytes = mask_bytes_fc(pl, B, L);
  }
  return 0;
}

int32_t salt_layer_forward(const salt_layer_desc* desc, const salt_qparams* prm,
                           const salt_events_in* in, const salt_events_out* out,
                           const salt_layer_result* res, void* d_workspace,
                           size_t workspace_bytes, void* stream) {
  int32_t rc = layer_forward(desc, prm, in, out, res, d_workspace, workspace_bytes, nullptr, 0);
  if (rc) return rc;
  return layer_forward(desc, prm, in, out, res, d_workspace, workspace_bytes,
                       (hipStream_t)stream, 1);
}

int32_t salt_layer_trace(const salt_layer_desc* desc, const salt_qparams* prm,
                         const salt_events_in* in, int32_t steps, int32_t* d_v_steps,
                         float* d_event_ms, uint8_t* d_flags, void* stream) {
  int32_t rc = check_common(desc, prm);
  if (rc) return rc;
  if (!in) return fail(-1, "null events descriptor");
  const int B = in->B, L = in->L;
  if (B < 0 || L < 0) return fail(-1, "invalid batch shape B=%d L=%d", B, L);
  if (B > 65535) return fail(-1, "batch of %d streams above 65535", B);
  const bool conv = desc->kind == SALT_LAYER_CONV;
  TraceArgs a;
  memset(&a, 0, sizeof(a));
  a.conv = conv;
  if (conv) {
    ConvPlan pl;
    if ((rc = plan_conv(desc, prm, 1, false, false, &pl))) return rc;
    a.IC = desc->ic; a.Hin = desc->h_in; a.Win = desc->w_in; a.K = desc->k; a.S = desc->s;
    a.P = desc->p; a.H = pl.H; a.W = pl.W; a.mql = desc->max_queue_len;
    a.n = desc->oc * pl.HW;
    if (desc->max_queue_len < 1) return fail(-1, "max_queue_len must be at least 1");
    if (steps != desc->max_queue_len)
      return fail(-1, "conv trace: steps=%d must equal max_queue_len=%d", steps,
                  desc->max_queue_len);
  } else {
    a.n_in = desc->n_in; a.n_out = desc->n_out;
    a.n = desc->n_out;
    if (steps != L) return fail(-1, "FC trace: steps=%d must equal the stream length L=%d", steps, L);
  }
  a.steps = steps;
  if (B == 0 || a.n == 0 || steps == 0) return 0;
  if (!in->d_n_real || (L > 0 && (!in->d_times || !in->d_src)))
    return fail(-1, "input events missing");
  if (!d_v_steps || !d_event_ms || !d_flags) return fail(-1, "trace output buffers missing");
  a.sat = prm->overflow_mode == SALT_SATURATE;
  a.qz = make_quant(prm);
  a.table = prm->d_decay_table;
  a.q = prm->d_q;
  a.q_bits = prm->q_bits;
  a.L = L; a.times = in->d_times; a.src = in->d_src; a.n_real = in->d_n_real;
  a.v_steps = d_v_steps; a.event_ms = d_event_ms; a.flags = d_flags;
  HIP_TRY(launch_trace(a, B, (hipStream_t)stream));
  return 0;
}

int32_t salt_stream_hash(const float* d_times, const int32_t* d_src, const int32_t* d_n,
                         int32_t B, int32_t cap, uint64_t* d_hash, void* stream) {
  if (B < 0 || cap < 0 || !d_n || !d_hash || (cap > 0 && (!d_times || !d_src)))
    return fail(-1, "invalid hash arguments");
  if (B == 0) return 0;
  hipLaunchKernelGGL(stream_hash_kernel, dim3(B), dim3(256), 0, (hipStream_t)stream, d_times,
                     d_src, d_n, cap, d_hash);
  HIP_TRY(hipGetLastError());
  return 0;
}

}  // extern "C"

namespace {

// Layer i's input: the caller's events for i = 0, else layer i-1's output stream.
salt_events_in network_input(const salt_events_in* in, const salt_events_out* outs, int i) {
  if (i == 0) return *in;
  salt_events_in e;
  e.B = in->B;
  e.L = outs[i - 1].cap;
  e.d_times = outs[i - 1].d_times;
  e.d_src = outs[i - 1].d_src;
  e.d_n_real = outs[i - 1].d_n;
  return e;
}

int64_t layer_inputs(const salt_layer_desc* d) {
  return d->kind == SALT_LAYER_CONV ? (int64_t)d->ic * d->h_in * d->w_in : d->n_in;
}

int64_t layer_neurons(const salt_layer_desc* d) {
  if (d->kind != SALT_LAYER_CONV) return d->n_out;
  const int64_t H = (d->h_in + 2 * d->p - d->k) / d->s + 1;
  const int64_t W = (d->w_in + 2 * d->p - d->k) / d->s + 1;
  return d->oc * H * W;
}

int32_t check_chain(int32_t n, const salt_layer_desc* descs, const salt_qparams* prms) {
  if (n < 1 || !descs || !prms) return fail(-1, "network: need at least one layer");
  for (int i = 1; i < n; ++i)
    if (layer_inputs(&descs[i]) != layer_neurons(&descs[i - 1]))
      return fail(-1, "network: layer %d takes %lld inputs, layer %d has %lld neurons", i,
                  (long long)layer_inputs(&descs[i]), i - 1,
                  (long long)layer_neurons(&descs[i - 1]));
  return 0;
}

}  // namespace

extern "C" {

int32_t salt_network_workspace_size(int32_t n_layers, const salt_layer_desc* descs,
                                    const salt_qparams* prms, int32_t B, int32_t L,
                                    int32_t want_neuron_extremes, size_t* bytes) {
  int32_t rc = check_chain(n_layers, descs, prms);
  if (rc) return rc;
  if (!bytes) return fail(-1, "null size pointer");
  size_t most = 0;
  for (int i = 0; i < n_layers; ++i) {
    size_t b = 0;
    const int32_t Li = i == 0 ? L : descs[i - 1].max_out_spikes;
    rc = salt_layer_workspace_size(&descs[i], &prms[i], B, Li, want_neuron_extremes, &b);
    if (rc) return rc;
    most = std::max(most, b);
  }
  *bytes = most;
  return 0;
}

int32_t salt_network_forward(int32_t n_layers, const salt_layer_desc* descs,
                             const salt_qparams* prms, const salt_events_in* in,
                             const salt_events_out* outs, const salt_layer_result* results,
                             void* d_workspace, size_t workspace_bytes, void* stream) {
  int32_t rc = check_chain(n_layers, descs, prms);
  if (rc) return rc;
  if (!in || !outs || !results) return fail(-1, "null events or result descriptors");
  for (int i = 0; i < n_layers; ++i) {
    const salt_events_in e = network_input(in, outs, i);
    if ((rc = layer_forward(&descs[i], &prms[i], &e, &outs[i], &results[i], d_workspace,
                            workspace_bytes, nullptr, 0)))
      return rc;
  }
  for (int i = 0; i < n_layers; ++i) {
    const salt_events_in e = network_input(in, outs, i);
    if ((rc = layer_forward(&descs[i], &prms[i], &e, &outs[i], &results[i], d_workspace,
                            workspace_bytes, (hipStream_t)stream, 1)))
      return rc;
  }
  return 0;
}

}  // extern "C"

// ------------------------------------------------------------------ static scratch

namespace {

// Workspace of salt_layer_forward_static: one array per device, held until the process
// ends.  In host code `scratch` names a host-side stand-in, not device memory, so its
// device address is looked up once per device (with that device current) and only that
// address is ever passed to kernels or fills.
constexpr size_t kScratchBytes = SALT_STATIC_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

int32_t scratch_address(void** out) {
  static std::mutex mu;
  static std::map<int, void*> per_device;
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  std::lock_guard<std::mutex> g(mu);
  auto it = per_device.find(dev);
  if (it == per_device.end()) {
    void* ptr = nullptr;
    HIP_TRY(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    if (!ptr) return fail(-2, "hipGetSymbolAddress(scratch) gave a null address");
    it = per_device.emplace(dev, ptr).first;
  }
  *out = it->second;
  return 0;
}

}  // namespace

extern "C" {

int32_t salt_layer_forward_static(const salt_layer_desc* desc, const salt_qparams* prm,
                                  const salt_events_in* in, const salt_events_out* out,
                                  const salt_layer_result* res, void* stream) {
  if (!in) return fail(-1, "null events descriptor");
  size_t need = 0;
  int32_t rc = salt_layer_workspace_size(desc, prm, in->B, in->L,
                                         res && res->d_v_min != nullptr, &need);
  if (rc) return rc;
  if (need > kScratchBytes)
    return fail(-1,
                "salt_layer_forward_static: this layer and batch need %zu bytes of scratch, "
                "above the static maximum of %zu; use salt_layer_forward with a workspace",
                need, kScratchBytes);
  void* ptr = nullptr;
  if ((rc = scratch_address(&ptr))) return rc;
  if ((rc = layer_forward(desc, prm, in, out, res, ptr, kScratchBytes, nullptr, 0))) return rc;
  return layer_forward(desc, prm, in, out, res, ptr, kScratchBytes, (hipStream_t)stream, 1);
}

}  // extern "C"
