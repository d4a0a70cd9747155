// libsalt_hip.so: MI355X (gfx950, CDNA4) kernels and C-ABI for the integer
// event-by-event forward pass of salt_core/quant.  The exported entry points are
// declared, with their reference counterparts, in include/salt_hip.h.
//
// Work decomposition.  A stream is strictly sequential per neuron, so parallelism
// comes from streams (batch) and from the neurons one event touches.  Each layer is
// split into partitions; one 64-lane wavefront owns one (stream, partition) pair and
// consumes that stream's events in order:
//   conv: partition = a group of output channels x a band of output rows.  Membrane
//         registers, the per-position last-update time and queue counters live in
//         LDS.  Per event, lanes 0..NC^2-1 resolve the NC x NC candidate positions
//         (decay code, queue capacity), the update lanes fetch them with ds_bpermute,
//         and every (channel, position) update is one lane.  No barrier is needed:
//         a wave's LDS operations complete in program order.
//   FC:   partition = a slice of 64*NPL neurons; registers live in VGPRs, weight
//         columns come from a transposed (n_in, n_out) copy in global memory.
// When one partition holds the whole layer the wave writes the spike stream itself:
// spikes of one event come out lane-ordered, which is ascending neuron id, the order
// of salt_core/stream.py:29-30.  Otherwise each partition ORs per-event spike bitmasks
// (bit order = neuron order) and a compaction kernel turns them into the stream.
//
// Fixed point.  The register update restates salt_core/quant/scan.py:22-52:
//   D = A*(V >> f_a) + ((A*(V & (2^f_a-1)) + c) >> f_a)     (fixed_point.py:47-65)
// with 24-bit multiplies (v_mul_i32_i24 / v_mul_u32_u24, full rate) whenever the
// register width allows (i_V + f_V - f_a <= 24), and 32-bit multiplies otherwise.
// The identity column (dt == 0) uses A = 2^f_a, which the same formula maps to V.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

#include "salt_hip.h"

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

constexpr int kWave = 64;
constexpr int kMaxIt = 8;                 // update iterations per event (<= 512 items)
constexpr float kPadTime = 1e12f;         // salt_core/stream.py:13
constexpr int kLdsMax = 160 * 1024;       // gfx950 LDS per workgroup
constexpr int kLdsPartBudget = 64 * 1024; // per partitioned wave (>= 2 waves per CU)
constexpr int kMaxPartPositions = 32767;  // packed position index must fit 15 bits

// ------------------------------------------------------------------ device helpers

struct Quant {
  int fa, fV, wbits, rc, sat, half;
  int n_table;  // extended table in LDS has n_table + 2 entries
  int vth_kind, vth_scalar;
  const int32_t* vth;
};

// Decay multiply with rounding, salt_core/quant/fixed_point.py:47-65.
template <bool FAST24>
__device__ __forceinline__ int32_t decay_mul(int32_t v, int32_t a, int fa, int rc) {
  int32_t hi = v >> fa;
  uint32_t lo = (uint32_t)v & ((1u << fa) - 1u);
  uint32_t t1 = __umul24((uint32_t)a, lo) + (uint32_t)rc;
  int32_t t2 = (int32_t)(t1 >> fa);
  return FAST24 ? __mul24(a, hi) + t2 : a * hi + t2;
}

// Write-back into the (i_V + f_V)-bit register, salt_core/quant/fixed_point.py:68-90.
__device__ __forceinline__ int32_t fit_bits(int32_t u, const Quant& qz) {
  if (qz.sat) return min(max(u, -qz.half), qz.half - 1);
  const unsigned sh = 32u - (unsigned)qz.wbits;
  return (int32_t)((uint32_t)u << sh) >> sh;
}

// Decay-table index for a float32 dt holding integer ms, salt_core/quant/codes.py:87-105:
// 0 -> identity slot, 1..n -> table, > n -> the zero slot n + 1.
__device__ __forceinline__ int decay_index(float dt, int n_table) {
  if (!(dt > 0.0f)) return 0;  // dt == 0 (negative/NaN cannot occur for valid input)
  if (dt > (float)n_table) return n_table + 1;
  return (int)dt;
}

__device__ __forceinline__ int floordiv_pos(int a, int s) {  // s > 0
  return a >= 0 ? a / s : -((-a + s - 1) / s);
}

__device__ __forceinline__ int wave_min(int v) {
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ int wave_max(int v) {
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ int wave_sum(int v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
// Exclusive prefix sum over the 64 lanes.
__device__ __forceinline__ int wave_excl_scan(int v, int lane) {
  int incl = v;
  for (int o = 1; o < 64; o <<= 1) {
    int t = __shfl_up(incl, o);
    if (lane >= o) incl += t;
  }
  return incl - v;
}

__device__ __forceinline__ uint64_t lanemask_lt(int lane) {
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

__device__ __forceinline__ int rdlane(int v, int lane) {
  return __builtin_amdgcn_readlane(v, lane);
}
__device__ __forceinline__ float rdlanef(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Extended decay table: [0] = 2^f_a (identity), [1..n] = table, [n+1] = 0.
__device__ void load_ext_table(int32_t* ext, const int32_t* table, int n_table, int fa,
                               int lane) {
  for (int i = lane; i < n_table + 2; i += kWave) {
    int32_t v;
    if (i == 0) v = 1 << fa;
    else if (i <= n_table) v = table[i - 1];
    else v = 0;
    ext[i] = v;
  }
}

__global__ void fill_i32_kernel(int32_t* p, int32_t value, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = value;
}

// ------------------------------------------------------------------ conv kernel

struct ConvArgs {
  // geometry
  int IC, Hin, Win, HWin, OC, K, S, P, H, W, HW, NC, NC2, WPO, mql;
  // partition: G channels x R rows per wave
  int G, n_og, R;
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

__device__ __forceinline__ int32_t load_code_bits(const void* p, size_t i, int bits) {
  if (bits == 8) return (int32_t) static_cast<const int8_t*>(p)[i];
  if (bits == 16) return (int32_t) static_cast<const int16_t*>(p)[i];
  return static_cast<const int32_t*>(p)[i];
}

template <typename T>
__device__ __forceinline__ T lds_at(char* base, int byte_off) {
  return *reinterpret_cast<T*>(base + byte_off);
}
template <typename T>
__device__ __forceinline__ void lds_put(char* base, int byte_off, T v) {
  *reinterpret_cast<T*>(base + byte_off) = v;
}

// LDS layout (4-byte words): trash[64] | ext[n_table+2] | vthc[G] | qs[G*IC*K*K] |
// V[G*R*W] | tl[R*W] | cnt[R*W] | (EXT) mn[G*R*W] | mx[G*R*W] | (VTHN) th[G*R*W]
constexpr int kConvFixedWords = 64;

size_t conv_lds_words(int n_table, int G, int IC, int K, int R, int W, bool ext, bool vthn) {
  return (size_t)kConvFixedWords + (size_t)(n_table + 2) + (size_t)G +
         (size_t)G * IC * K * K + (size_t)G * R * W * (1 + (ext ? 2 : 0) + (vthn ? 1 : 0)) +
         2 * (size_t)R * W;
}

// One wave per (stream, partition).  Per event, the updates are the valid candidate
// rectangle (ny x nx positions) times the partition's channels, compacted onto lanes:
// item u -> channel u / (ny*nx), position u % (ny*nx) (exact float-reciprocal division).
// The iteration body has no divergent branches: lanes without an update read from a
// safe address and write to their own trash word.  All LDS reads of an event are
// issued before their results are needed (two dependent round trips: registers, codes,
// last times, counts, then decay codes).  NIT bounds the iterations per event.
template <bool FAST24, bool EXT, bool VTHN, int NIT>
__global__ void __launch_bounds__(64) conv_layer_kernel(ConvArgs a) {
  extern __shared__ int32_t smem[];
  const int lane = threadIdx.x;
  const int b = blockIdx.y;
  const int og = blockIdx.x % a.n_og;
  const int rb = blockIdx.x / a.n_og;
  const int oc0 = og * a.G;
  const int ocn = min(a.G, a.OC - oc0);
  const int r0 = rb * a.R;
  const int rn = min(a.R, a.H - r0);
  const int W = a.W;
  const int PW = rn * W;  // positions in this partition
  const int KK = a.K * a.K;
  const Quant& qz = a.qz;

  int32_t* ext = smem + kConvFixedWords;
  int32_t* vthc = ext + (qz.n_table + 2);
  int32_t* qs = vthc + a.G;
  int32_t* Vs = qs + a.G * a.IC * KK;
  float* tl = reinterpret_cast<float*>(Vs + a.G * a.R * W);
  int32_t* cnt = reinterpret_cast<int32_t*>(tl + a.R * W);
  int32_t* mn = cnt + a.R * W;
  int32_t* mx = mn + (EXT ? a.G * a.R * W : 0);
  int32_t* th = mx + (EXT ? a.G * a.R * W : 0);

  load_ext_table(ext, a.table, qz.n_table, qz.fa, lane);
  for (int i = lane; i < a.G; i += kWave)
    vthc[i] = qz.vth_kind == SALT_VTH_PER_CHANNEL ? qz.vth[min(oc0 + i, a.OC - 1)] : qz.vth_scalar;
  for (int i = lane; i < ocn * a.IC * KK; i += kWave)
    qs[i] = load_code_bits(a.q, (size_t)oc0 * a.IC * KK + i, a.q_bits);
  for (int i = lane; i < ocn * PW; i += kWave) {
    Vs[i] = 0;
    if (EXT) { mn[i] = 0; mx[i] = 0; }
    if (VTHN) {
      const int ocl = i / PW;
      th[i] = qz.vth[(oc0 + ocl) * a.HW + r0 * W + (i - ocl * PW)];
    }
  }
  for (int i = lane; i < PW; i += kWave) { tl[i] = 0.0f; cnt[i] = 0; }
  __syncthreads();

  const int L = a.L;
  const int nr = a.n_real[b];
  const int n_eff = nr < 0 ? 0 : (nr < L ? nr : L);
  const float* tb = a.times + (size_t)b * L;
  const int32_t* sb = a.src + (size_t)b * L;
  const bool has_vth = qz.vth_kind != SALT_VTH_NONE;
  const float tab_top = (float)(qz.n_table + 1);
  const uint32_t qfV = (uint32_t)qz.fV;

  char* const lds = reinterpret_cast<char*>(smem);
  const int trash4 = lane * 4;  // this lane's trash word
  const int ext4 = (int)(reinterpret_cast<char*>(ext) - lds);
  const int vthc4 = (int)(reinterpret_cast<char*>(vthc) - lds);
  const int qs4 = (int)(reinterpret_cast<char*>(qs) - lds);
  const int vs4 = (int)(reinterpret_cast<char*>(Vs) - lds);
  const int tl4 = (int)(reinterpret_cast<char*>(tl) - lds);
  const int cnt4 = (int)(reinterpret_cast<char*>(cnt) - lds);
  const int mn4 = (int)(reinterpret_cast<char*>(mn) - lds);
  const int mx4 = (int)(reinterpret_cast<char*>(mx) - lds);
  const int th4 = (int)(reinterpret_cast<char*>(th) - lds);
  const int PW4 = PW * 4, ICKK4 = a.IC * KK * 4, SK4 = a.S * a.K * 4, S4 = a.S * 4;
  float uf[NIT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) uf[it] = (float)(it * kWave + lane) + 0.5f;

  int vmin_l = 0, vmax_l = 0;
  int out_base = 0;

  for (int base = 0; base < n_eff; base += kWave) {
    // Decode 64 events at once, one per lane (connectivity/conv.py:15-43).
    const int j = base + lane;
    const bool ok = j < n_eff;
    const float tv = ok ? tb[j] : 0.0f;
    const int sv = ok ? sb[j] : -1;
    bool rel = ok && sv >= 0;
    int c = 0, y = 0, x = 0;
    if (rel) {
      c = sv / a.HWin;
      const int rem = sv - c * a.HWin;
      y = rem / a.Win;
      x = rem - y * a.Win;
      c = min(c, a.IC - 1);  // memory safety only; the host rejects such ids
    }
    const int oy0 = floordiv_pos(y + a.P - a.K + a.S, a.S);  // ceil((y+P-K+1)/S)
    const int ox0 = floordiv_pos(x + a.P - a.K + a.S, a.S);
    const int oyA = max(oy0, r0), oyB = min((y + a.P) / a.S, r0 + rn - 1);
    const int oxA = max(ox0, 0), oxB = min((x + a.P) / a.S, W - 1);
    rel = rel && oyA <= oyB && oxA <= oxB;
    // Packed per-event fields: rectangle origin and size in candidate units, the
    // partition position of its first cell, and the weight-code offset of that cell.
    const int dyA = oyA - oy0, dxA = oxA - ox0;
    const int rect = dyA | (dxA << 8) | ((oyB - oyA + 1) << 16) | ((oxB - oxA + 1) << 24);
    const int pbase = (oyA - r0) * W + oxA;
    const int qe4 = (c * KK + (y + a.P - oyA * a.S) * a.K + (x + a.P - oxA * a.S)) * 4;
    uint64_t todo = __ballot(rel);

    while (todo) {
      const int e = __builtin_ctzll(todo);
      todo &= todo - 1;
      const float te = rdlanef(tv, e);
      const int rect_e = rdlane(rect, e);
      const int pbase_e = rdlane(pbase, e);
      const int qe4_e = rdlane(qe4, e);
      const int ny = (rect_e >> 16) & 0xFF, nx = (int)((uint32_t)rect_e >> 24);
      const int area = ny * nx;
      const int items = ocn * area;
      const int nit_e = (items + kWave - 1) >> 6;
      const float inv_area = __builtin_amdgcn_rcpf((float)area);
      const float inv_nx = __builtin_amdgcn_rcpf((float)nx);

      // Round trip 1: register, code, threshold, last-update time, queue count.
      int v[NIT], qv[NIT], vt[NIT], cb[NIT], lp[NIT], nl4[NIT], ocv[NIT], pv[NIT];
      int mnv[NIT], mxv[NIT];
      float tlv[NIT];
      bool val[NIT];
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        if (it < nit_e) {
          // All index products are small: 24-bit multiplies (full rate).
          const int u = it * kWave + lane;
          val[it] = u < items;
          const int oc = min((int)(uf[it] * inv_area), ocn - 1);
          const int p = u - __mul24(oc, area);
          const int dy = (int)(((float)p + 0.5f) * inv_nx);
          const int dx = p - __mul24(dy, nx);
          const int lp_raw = pbase_e + __mul24(dy, W) + dx;
          const int q4_raw = __mul24(oc, ICKK4) - __mul24(dy, SK4) - __mul24(dx, S4) + qe4_e;
          lp[it] = val[it] ? lp_raw : 0;  // lanes without an item read in-range words
          ocv[it] = oc;
          pv[it] = p;
          nl4[it] = __mul24(oc, PW4) + lp[it] * 4;
          const int q4 = val[it] ? q4_raw : 0;
          const int vaddr = val[it] ? vs4 + nl4[it] : trash4;
          v[it] = lds_at<int32_t>(lds, vaddr);
          qv[it] = lds_at<int32_t>(lds, qs4 + q4);
          vt[it] = VTHN ? lds_at<int32_t>(lds, val[it] ? th4 + nl4[it] : trash4)
                        : lds_at<int32_t>(lds, vthc4 + (val[it] ? oc : 0) * 4);
          tlv[it] = lds_at<float>(lds, tl4 + lp[it] * 4);
          cb[it] = lds_at<int32_t>(lds, cnt4 + lp[it] * 4);
          if (EXT) {
            mnv[it] = lds_at<int32_t>(lds, val[it] ? mn4 + nl4[it] : trash4);
            mxv[it] = lds_at<int32_t>(lds, val[it] ? mx4 + nl4[it] : trash4);
          }
        }
      }
      // Round trip 2: decay codes (salt_core/quant/codes.py:87-105; index 0 = identity).
      int A[NIT];
#pragma unroll
      for (int it = 0; it < NIT; ++it)
        if (it < nit_e)
          A[it] = lds_at<int32_t>(lds, ext4 + 4 * (int)fminf(fmaxf(te - tlv[it], 0.0f), tab_top));
      // Update (salt_core/quant/scan.py:22-52), write back, emit spikes.
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        if (it < nit_e) {
          const bool act = val[it] && cb[it] < a.mql;  // a full queue drops the event
          const int32_t d = decay_mul<FAST24>(v[it], A[it], qz.fa, qz.rc);
          const int32_t u = (int32_t)((uint32_t)d + ((uint32_t)qv[it] << qfV));
          const int32_t f = fit_bits(u, qz);
          const bool fire = act && has_vth && f >= vt[it];
          lds_put<int32_t>(lds, act ? vs4 + nl4[it] : trash4, fire ? 0 : f);
          const int um = act ? u : 0;
          vmin_l = min(vmin_l, um);
          vmax_l = max(vmax_l, um);
          if (EXT) {
            lds_put<int32_t>(lds, act ? mn4 + nl4[it] : trash4, min(mnv[it], u));
            lds_put<int32_t>(lds, act ? mx4 + nl4[it] : trash4, max(mxv[it], u));
          }
          const uint64_t bal = __ballot(fire);
          if (bal) {
            const int neuron = (oc0 + ocv[it]) * a.HW + r0 * W + lp[it];
            if (a.direct) {
              if (fire) {
                const int idx = out_base + __popcll(bal & lanemask_lt(lane));
                if (idx < a.cap) {
                  a.out_t[(size_t)b * a.cap + idx] = te;
                  a.out_s[(size_t)b * a.cap + idx] = neuron;
                }
              }
              out_base += __popcll(bal);
            } else if (fire) {
              // Candidate index within the event's NC x NC grid = mask bit.
              const int dy = pv[it] / nx, dx = pv[it] - (pv[it] / nx) * nx;
              const int r = ((rect_e & 0xFF) + dy) * a.NC + (((rect_e >> 8) & 0xFF) + dx);
              const size_t w = ((size_t)b * L + base + e) * (size_t)(a.OC * a.WPO) +
                               (size_t)(oc0 + ocv[it]) * a.WPO + (r >> 5);
              atomicOr(&a.masks[w], 1u << (r & 31));
            }
          }
        }
      }
      // Commit the touched positions' queue count and last-update time (channel-0
      // items, which are the first `area` lanes of iteration 0).
      {
        const bool commit = lane < area;
        lds_put<int32_t>(lds, commit ? cnt4 + lp[0] * 4 : trash4, cb[0] + 1);
        lds_put<float>(lds, (commit && cb[0] < a.mql) ? tl4 + lp[0] * 4 : trash4, te);
      }
      asm volatile("" ::: "memory");  // keep this event's LDS traffic before the next one's
    }
  }

  // Catch-up column: decay to the last real input time T (connectivity/conv.py:102-125).
  // An empty position's catch-up has dt = 0; the identity columns after it repeat V.
  const float T = n_eff > 0 ? tb[n_eff - 1] : 0.0f;
  int maxcnt = 0;
  for (int i = lane; i < PW; i += kWave) maxcnt = max(maxcnt, cnt[i]);
  for (int li = lane; li < ocn * PW; li += kWave) {
    const int ocl = li / PW;
    const int lpp = li - ocl * PW;
    const int cbv = cnt[lpp];
    int32_t vv = Vs[li];
    if (cbv < a.mql) {
      const float dt = cbv > 0 ? T - tl[lpp] : 0.0f;
      const int A = ext[(int)fminf(fmaxf(dt, 0.0f), tab_top)];
      vv = decay_mul<FAST24>(vv, A, qz.fa, qz.rc);  // |D| <= |V|: in range, cannot fire
      vmin_l = min(vmin_l, vv);
      vmax_l = max(vmax_l, vv);
      if (EXT) {
        mn[li] = min(mn[li], vv);
        mx[li] = max(mx[li], vv);
      }
    }
    const size_t ng = (size_t)b * (a.OC * a.HW) + (size_t)(oc0 + ocl) * a.HW + r0 * W + lpp;
    if (a.v_final) a.v_final[ng] = vv;
    if (EXT) {
      a.v_min[ng] = mn[li];
      a.v_max[ng] = mx[li];
    }
  }
  vmin_l = wave_min(vmin_l);
  vmax_l = wave_max(vmax_l);
  maxcnt = wave_max(maxcnt);
  const int ovf = (vmin_l < -qz.half || vmax_l > qz.half - 1) ? 1 : 0;
  if (a.direct) {
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
  } else if (lane == 0) {
    atomicMin(&a.stats[b * 4 + 0], vmin_l);
    atomicMax(&a.stats[b * 4 + 1], vmax_l);
    atomicMax(&a.stats[b * 4 + 2], maxcnt + 1);
    atomicOr(&a.stats[b * 4 + 3], ovf);
  }
}

// ------------------------------------------------------------------ FC kernel

struct FcArgs {
  int n_in, n_out, words;  // words: 32-bit mask words per event
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

// One wave = one stream x one slice of 64*NPL neurons, neuron = n0 + k*64 + lane.
// connectivity/fc.py:20-33, 54-61; layers/fc.py:84-124.  WLDS: the slice's weight
// columns (n_in x slice, native width) are staged in LDS; otherwise they are read from the
// transposed global copy, one event ahead.
template <typename QT, int NPL, bool FAST24, bool WLDS>
__global__ void __launch_bounds__(64) fc_layer_kernel(FcArgs a) {
  extern __shared__ int32_t dyn[];
  const int lane = threadIdx.x;
  const int b = blockIdx.y;
  const int n0 = blockIdx.x * (kWave * NPL);
  const int sw = min(kWave * NPL, a.n_out - n0);  // neurons in this slice
  const Quant& qz = a.qz;
  int32_t* tab = dyn;
  QT* wl = reinterpret_cast<QT*>(dyn + (qz.n_table + 2));
  const QT* qt = static_cast<const QT*>(a.qt);
  load_ext_table(tab, a.table, qz.n_table, qz.fa, lane);
  if (WLDS)
    for (int i = lane; i < a.n_in * sw; i += kWave) {
      const int r = i / sw;
      wl[i] = qt[(size_t)r * a.n_out + n0 + (i - r * sw)];
    }
  __syncthreads();

  int32_t V[NPL], mn[NPL], mx[NPL], vth[NPL];
  bool nv[NPL];
#pragma unroll
  for (int k = 0; k < NPL; ++k) {
    const int n = n0 + k * kWave + lane;
    nv[k] = n < a.n_out;
    V[k] = 0;
    mn[k] = 0;
    mx[k] = 0;
    vth[k] = qz.vth_kind == SALT_VTH_SCALAR ? qz.vth_scalar
             : (qz.vth_kind != SALT_VTH_NONE && nv[k]) ? qz.vth[n] : 0;
  }
  const bool has_vth = qz.vth_kind != SALT_VTH_NONE;
  const float tab_top = (float)(qz.n_table + 1);
  const int L = a.L;
  const int nr = a.n_real[b];
  const int n_eff = nr < 0 ? 0 : (nr < L ? nr : L);
  const float* tb = a.times + (size_t)b * L;
  const int32_t* sb = a.src + (size_t)b * L;
  float t_prev = 0.0f;  // the first event is compared with t = 0 (fc.py:30)
  int out_base = 0;

  for (int base = 0; base < n_eff; base += kWave) {
    const int j = base + lane;
    const bool ok = j < n_eff;
    const float tv = ok ? tb[j] : 0.0f;
    const int sv = ok ? min(max(sb[j], 0), a.n_in - 1) : 0;
    const int ne = min(kWave, n_eff - base);
    int32_t qn[NPL];
    if (!WLDS) {
      const int s0 = rdlane(sv, 0);
#pragma unroll
      for (int k = 0; k < NPL; ++k)
        qn[k] = nv[k] ? (int32_t)qt[(size_t)s0 * a.n_out + n0 + k * kWave + lane] : 0;
    }
    for (int e = 0; e < ne; ++e) {
      const int se = rdlane(sv, e);
      int32_t qc[NPL];
      if (WLDS) {
#pragma unroll
        for (int k = 0; k < NPL; ++k) qc[k] = nv[k] ? (int32_t)wl[se * sw + k * kWave + lane] : 0;
      } else {
#pragma unroll
        for (int k = 0; k < NPL; ++k) qc[k] = qn[k];
        if (e + 1 < ne) {
          const int s1 = rdlane(sv, e + 1);
#pragma unroll
          for (int k = 0; k < NPL; ++k)
            qn[k] = nv[k] ? (int32_t)qt[(size_t)s1 * a.n_out + n0 + k * kWave + lane] : 0;
        }
      }
      const float te = rdlanef(tv, e);
      const int A = tab[(int)fminf(fmaxf(te - t_prev, 0.0f), tab_top)];
      t_prev = te;
#pragma unroll
      for (int k = 0; k < NPL; ++k) {
        bool fire = false;
        if (nv[k]) {
          const int32_t d = decay_mul<FAST24>(V[k], A, qz.fa, qz.rc);
          const int32_t u = (int32_t)((uint32_t)d + ((uint32_t)qc[k] << qz.fV));
          const int32_t f = fit_bits(u, qz);
          fire = has_vth && f >= vth[k];
          V[k] = fire ? 0 : f;
          mn[k] = min(mn[k], u);
          mx[k] = max(mx[k], u);
        }
        const uint64_t bal = __ballot(fire);
        if (a.direct) {
          if (bal) {
            if (fire) {
              const int idx = out_base + __popcll(bal & lanemask_lt(lane));
              if (idx < a.cap) {
                a.out_t[(size_t)b * a.cap + idx] = te;
                a.out_s[(size_t)b * a.cap + idx] = n0 + k * kWave + lane;
              }
            }
            out_base += __popcll(bal);
          }
        } else {
          const int w0 = (n0 + k * kWave) >> 5;
          if (lane < 2 && w0 + lane < a.words)
            a.masks[((size_t)b * L + base + e) * a.words + w0 + lane] =
                lane ? (uint32_t)(bal >> 32) : (uint32_t)bal;
        }
      }
    }
  }
  // Pad columns (j >= n_real) are identity with code 0 (fc.py:32, :60-61): U = V.
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

// ------------------------------------------------------------------ compaction

struct CompactArgs {
  int conv;                      // 1: conv bit layout, 0: FC (neuron = word*32 + bit)
  int words, WPO, NC, OC, HW, W, HWin, Win, K, S, P;
  int L;
  const float* times;
  const int32_t* src;
  const int32_t* n_real;
  const uint32_t* masks;
  int cap, fill_pads;
  float* out_t;
  int32_t* out_s;
  int32_t* out_n;
};

// Spike bitmasks -> ordered stream.  One wave per stream; lane = event within a chunk
// of 64.  Words are in neuron order and bits within a word too, so walking them gives
// the (event, neuron) order of salt_core/stream.py:24-46.
__global__ void __launch_bounds__(64) compact_kernel(CompactArgs a) {
  const int lane = threadIdx.x;
  const int b = blockIdx.x;
  const int L = a.L;
  const int nr = a.n_real[b];
  const int n_eff = nr < 0 ? 0 : (nr < L ? nr : L);
  int out_base = 0;
  for (int base = 0; base < n_eff; base += kWave) {
    const int j = base + lane;
    const bool ok = j < n_eff;
    const uint32_t* m = a.masks + ((size_t)b * L + j) * a.words;
    int count = 0;
    if (ok)
      for (int w = 0; w < a.words; ++w) count += __popc(m[w]);
    const int excl = wave_excl_scan(count, lane);
    const int total = wave_sum(count);
    if (ok && count > 0) {
      int pos = out_base + excl;
      const float te = a.times[(size_t)b * L + j];
      int oy0 = 0, ox0 = 0;
      if (a.conv) {
        const int sv = a.src[(size_t)b * L + j];
        const int rem = sv % a.HWin;
        const int y = rem / a.Win, x = rem - (rem / a.Win) * a.Win;
        oy0 = floordiv_pos(y + a.P - a.K + a.S, a.S);
        ox0 = floordiv_pos(x + a.P - a.K + a.S, a.S);
      }
      for (int w = 0; w < a.words; ++w) {
        uint32_t bits = m[w];
        while (bits) {
          const int bit = __builtin_ctz(bits);
          bits &= bits - 1;
          int neuron;
          if (a.conv) {
            const int oc = w / a.WPO;
            const int r = (w - oc * a.WPO) * 32 + bit;
            const int dy = r / a.NC, dx = r - (r / a.NC) * a.NC;
            neuron = oc * a.HW + (oy0 + dy) * a.W + (ox0 + dx);
          } else {
            neuron = w * 32 + bit;
          }
          if (pos < a.cap) {
            a.out_t[(size_t)b * a.cap + pos] = te;
            a.out_s[(size_t)b * a.cap + pos] = neuron;
          }
          ++pos;
        }
      }
    }
    out_base += total;
  }
  if (lane == 0) a.out_n[b] = out_base;
  if (a.fill_pads)
    for (int i = min(out_base, a.cap) + lane; i < a.cap; i += kWave) {
      a.out_t[(size_t)b * a.cap + i] = kPadTime;
      a.out_s[(size_t)b * a.cap + i] = 0;
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

// ------------------------------------------------------------------ host side

struct ConvPlan {
  int H, W, HW, NC, NC2, WPO, G, R, n_og, n_rb, direct;
  size_t lds;
};

size_t conv_lds_bytes(const salt_layer_desc* d, int n_table, int G, int R, int W, bool ext,
                      bool vthn) {
  return conv_lds_words(n_table, G, d->ic, d->k, R, W, ext, vthn) * 4;
}

int32_t plan_conv(const salt_layer_desc* d, const salt_qparams* p, int B, bool ext,
                  ConvPlan* pl) {
  const bool vthn = p->v_th_kind == SALT_VTH_PER_NEURON;
  pl->H = (d->h_in + 2 * d->p - d->k) / d->s + 1;
  pl->W = (d->w_in + 2 * d->p - d->k) / d->s + 1;
  if (pl->H < 1 || pl->W < 1) return fail(-1, "conv geometry gives an empty output plane");
  pl->HW = pl->H * pl->W;
  pl->NC = (d->k - 1) / d->s + 1;
  pl->NC2 = pl->NC * pl->NC;
  if (pl->NC2 > kWave)
    return fail(-3, "conv: %d candidate positions per event (k=%d, s=%d) exceed 64", pl->NC2,
                d->k, d->s);
  pl->WPO = (pl->NC2 + 31) / 32;
  const int W = pl->W, H = pl->H, OC = d->oc;
  const int gmax_it = std::max(1, (kMaxIt * kWave) / pl->NC2);
  // Whole layer in one wave per stream when it fits and the batch alone fills the GPU.
  if (OC <= gmax_it && pl->HW <= kMaxPartPositions) {
    size_t lds = conv_lds_bytes(d, p->n_table, OC, H, W, ext, vthn);
    if ((lds <= 40 * 1024 && B >= 512) || (lds <= (size_t)kLdsMax && B >= 2048)) {
      pl->G = OC; pl->R = H; pl->n_og = 1; pl->n_rb = 1; pl->direct = 1; pl->lds = lds;
      return 0;
    }
  }
  // Partitioned: at most two update iterations per event, LDS within the budget, then
  // split channels further while the grid is smaller than ~2048 waves.
  int G = std::max(1, std::min(OC, (2 * kWave) / pl->NC2));
  for (;;) {
    int R = H;
    while (R > 1 && (conv_lds_bytes(d, p->n_table, G, R, W, ext, vthn) > (size_t)kLdsPartBudget ||
                     (size_t)R * W > (size_t)kMaxPartPositions))
      --R;
    if (conv_lds_bytes(d, p->n_table, G, R, W, ext, vthn) > (size_t)kLdsMax ||
        (size_t)R * W > (size_t)kMaxPartPositions) {
      if (G == 1) return fail(-3, "conv: one output row does not fit in LDS (w_out=%d)", W);
      G = (G + 1) / 2;
      continue;
    }
    const int n_og = (OC + G - 1) / G, n_rb = (H + R - 1) / R;
    if ((long)B * n_og * n_rb < 2048 && G > 1 && G * pl->NC2 > 32) {
      G = (G + 1) / 2;
      continue;
    }
    pl->G = G; pl->R = R; pl->n_og = n_og; pl->n_rb = n_rb;
    pl->direct = (n_og == 1 && n_rb == 1);
    pl->lds = conv_lds_bytes(d, p->n_table, G, R, W, ext, vthn);
    return 0;
  }
}

struct FcPlan {
  int npl, n_slices, words, direct;
};

int32_t plan_fc(const salt_layer_desc* d, FcPlan* pl) {
  int need = (d->n_out + kWave - 1) / kWave;
  int npl = 1;
  while (npl < need && npl < 16) npl *= 2;
  pl->npl = npl;
  pl->n_slices = (d->n_out + kWave * npl - 1) / (kWave * npl);
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
  q.sat = p->overflow_mode == SALT_SATURATE;
  q.half = 1 << (q.wbits - 1);
  q.n_table = p->n_table;
  q.vth_kind = p->v_th_kind;
  q.vth_scalar = p->v_th_scalar;
  q.vth = p->d_v_th;
  return q;
}

size_t mask_bytes_conv(const ConvPlan& pl, const salt_layer_desc* d, int B, int L) {
  return pl.direct ? 0 : (size_t)B * L * d->oc * pl.WPO * 4;
}
size_t mask_bytes_fc(const FcPlan& pl, int B, int L) {
  return pl.direct ? 0 : (size_t)B * L * pl.words * 4;
}

int32_t fill(int32_t* p, int32_t v, size_t n, hipStream_t st) {
  if (n == 0) return 0;
  size_t blocks = std::min<size_t>((n + 255) / 256, 65536);
  hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)blocks), dim3(256), 0, st, p, v, n);
  HIP_TRY(hipGetLastError());
  return 0;
}

template <bool F24, bool EXT, bool VTHN, int NIT>
int32_t launch_conv_t(const ConvArgs& a, const ConvPlan& pl, int B, hipStream_t st) {
  auto kern = conv_layer_kernel<F24, EXT, VTHN, NIT>;
  static bool attr_set = false;  // per instantiation
  if (!attr_set) {
    HIP_TRY(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                kLdsMax));
    attr_set = true;
  }
  hipLaunchKernelGGL(kern, dim3(pl.n_og * pl.n_rb, B), dim3(kWave), pl.lds, st, a);
  HIP_TRY(hipGetLastError());
  return 0;
}

template <bool F24, bool EXT, bool VTHN>
int32_t launch_conv_n(const ConvArgs& a, const ConvPlan& pl, int B, hipStream_t st) {
  const int nit = (pl.G * pl.NC2 + kWave - 1) / kWave;
  if (nit <= 1) return launch_conv_t<F24, EXT, VTHN, 1>(a, pl, B, st);
  if (nit <= 2) return launch_conv_t<F24, EXT, VTHN, 2>(a, pl, B, st);
  if (nit <= 4) return launch_conv_t<F24, EXT, VTHN, 4>(a, pl, B, st);
  return launch_conv_t<F24, EXT, VTHN, kMaxIt>(a, pl, B, st);
}

int32_t launch_conv(const ConvArgs& a, const ConvPlan& pl, int B, bool f24, bool ext, bool vthn,
                    hipStream_t st) {
  if (f24) {
    if (ext) return vthn ? launch_conv_n<true, true, true>(a, pl, B, st)
                         : launch_conv_n<true, true, false>(a, pl, B, st);
    return vthn ? launch_conv_n<true, false, true>(a, pl, B, st)
                : launch_conv_n<true, false, false>(a, pl, B, st);
  }
  if (ext) return vthn ? launch_conv_n<false, true, true>(a, pl, B, st)
                       : launch_conv_n<false, true, false>(a, pl, B, st);
  return vthn ? launch_conv_n<false, false, true>(a, pl, B, st)
              : launch_conv_n<false, false, false>(a, pl, B, st);
}

constexpr size_t kFcWeightLds = 40 * 1024;  // stage FC weight slices up to this size

template <typename QT, int NPL, bool F24, bool WLDS>
int32_t launch_fc_t(const FcArgs& a, const FcPlan& pl, int B, hipStream_t st) {
  const int sw = std::min(kWave * NPL, a.n_out);
  size_t lds = (size_t)(a.qz.n_table + 2) * 4 + (WLDS ? (size_t)a.n_in * sw * sizeof(QT) : 0);
  if (lds > (size_t)kLdsMax) return fail(-3, "decay table too long for LDS");
  auto kern = fc_layer_kernel<QT, NPL, F24, WLDS>;
  static bool attr_set = false;
  if (!attr_set) {
    HIP_TRY(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                kLdsMax));
    attr_set = true;
  }
  hipLaunchKernelGGL(kern, dim3(pl.n_slices, B), dim3(kWave), lds, st, a);
  HIP_TRY(hipGetLastError());
  return 0;
}

template <typename QT, int NPL, bool F24>
int32_t launch_fc_w(const FcArgs& a, const FcPlan& pl, int B, hipStream_t st) {
  const size_t wbytes = (size_t)a.n_in * std::min(kWave * NPL, a.n_out) * sizeof(QT);
  if (wbytes + (size_t)(a.qz.n_table + 2) * 4 <= kFcWeightLds)
    return launch_fc_t<QT, NPL, F24, true>(a, pl, B, st);
  return launch_fc_t<QT, NPL, F24, false>(a, pl, B, st);
}

template <typename QT, bool F24>
int32_t launch_fc_npl(const FcArgs& a, const FcPlan& pl, int B, hipStream_t st) {
  switch (pl.npl) {
    case 1: return launch_fc_w<QT, 1, F24>(a, pl, B, st);
    case 2: return launch_fc_w<QT, 2, F24>(a, pl, B, st);
    case 4: return launch_fc_w<QT, 4, F24>(a, pl, B, st);
    case 8: return launch_fc_w<QT, 8, F24>(a, pl, B, st);
    default: return launch_fc_w<QT, 16, F24>(a, pl, B, st);
  }
}

template <typename QT>
int32_t launch_fc_q(const FcArgs& a, const FcPlan& pl, int B, bool f24, hipStream_t st) {
  return f24 ? launch_fc_npl<QT, true>(a, pl, B, st) : launch_fc_npl<QT, false>(a, pl, B, st);
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
    ConvPlan pl;
    rc = plan_conv(desc, prm, B, want_neuron_extremes != 0, &pl);
    if (rc) return rc;
    *bytes = mask_bytes_conv(pl, desc, B, L);
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
  hipStream_t st = (hipStream_t)stream;
  const Quant qz = make_quant(prm);
  const bool f24 = (prm->i_V + prm->f_V - prm->f_a) <= 24;

  if (desc->kind == SALT_LAYER_CONV) {
    ConvPlan pl;
    rc = plan_conv(desc, prm, B, ext, &pl);
    if (rc) return rc;
    const size_t need = mask_bytes_conv(pl, desc, B, L);
    if (workspace_bytes < need || (need && !d_workspace))
      return fail(-1, "workspace of %zu bytes below the %zu needed", workspace_bytes, need);
    ConvArgs a;
    a.IC = desc->ic; a.Hin = desc->h_in; a.Win = desc->w_in; a.HWin = desc->h_in * desc->w_in;
    a.OC = desc->oc; a.K = desc->k; a.S = desc->s; a.P = desc->p;
    a.H = pl.H; a.W = pl.W; a.HW = pl.HW; a.NC = pl.NC; a.NC2 = pl.NC2; a.WPO = pl.WPO;
    a.mql = desc->max_queue_len;
    a.G = pl.G; a.n_og = pl.n_og; a.R = pl.R;
    a.qz = qz; a.table = prm->d_decay_table; a.q = prm->d_q; a.q_bits = prm->q_bits;
    a.L = L; a.times = in->d_times; a.src = in->d_src; a.n_real = in->d_n_real;
    a.cap = out->cap; a.fill_pads = out->fill_pads; a.direct = pl.direct;
    a.out_t = out->d_times; a.out_s = out->d_src; a.out_n = out->d_n;
    a.v_final = res->d_v_final; a.v_min = res->d_v_min; a.v_max = res->d_v_max;
    a.stats = res->d_stats;
    a.masks = static_cast<uint32_t*>(d_workspace);
    if (!pl.direct) {
      if ((rc = fill(res->d_stats, 0, (size_t)B * 4, st))) return rc;
      if ((rc = fill(reinterpret_cast<int32_t*>(a.masks), 0, need / 4, st))) return rc;
    }
    rc = launch_conv(a, pl, B, f24, ext, prm->v_th_kind == SALT_VTH_PER_NEURON, st);
    if (rc) return rc;
    if (!pl.direct) {
      CompactArgs c;
      c.conv = 1; c.words = desc->oc * pl.WPO; c.WPO = pl.WPO; c.NC = pl.NC; c.OC = desc->oc;
      c.HW = pl.HW; c.W = pl.W; c.HWin = a.HWin; c.Win = desc->w_in; c.K = desc->k;
      c.S = desc->s; c.P = desc->p; c.L = L; c.times = in->d_times; c.src = in->d_src;
      c.n_real = in->d_n_real; c.masks = a.masks; c.cap = out->cap;
      c.fill_pads = out->fill_pads; c.out_t = out->d_times; c.out_s = out->d_src;
      c.out_n = out->d_n;
      hipLaunchKernelGGL(compact_kernel, dim3(B), dim3(kWave), 0, st, c);
      HIP_TRY(hipGetLastError());
    }
    return 0;
  }

  FcPlan pl;
  plan_fc(desc, &pl);
  const size_t need = mask_bytes_fc(pl, B, L);
  if (workspace_bytes < need || (need && !d_workspace))
    return fail(-1, "workspace of %zu bytes below the %zu needed", workspace_bytes, need);
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
  switch (prm->q_bits) {
    case 8: rc = launch_fc_q<int8_t>(a, pl, B, f24, st); break;
    case 16: rc = launch_fc_q<int16_t>(a, pl, B, f24, st); break;
    default: rc = launch_fc_q<int32_t>(a, pl, B, f24, st); break;
  }
  if (rc) return rc;
  if (!pl.direct) {
    CompactArgs c;
    memset(&c, 0, sizeof(c));
    c.conv = 0; c.words = pl.words; c.L = L; c.times = in->d_times; c.src = in->d_src;
    c.n_real = in->d_n_real; c.masks = a.masks; c.cap = out->cap;
    c.fill_pads = out->fill_pads; c.out_t = out->d_times; c.out_s = out->d_src;
    c.out_n = out->d_n;
    hipLaunchKernelGGL(compact_kernel, dim3(B), dim3(kWave), 0, st, c);
    HIP_TRY(hipGetLastError());
  }
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
