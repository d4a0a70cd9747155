/*
 * CPU oracle for the integer event-by-event forward pass of salt_core/quant.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path (tests/, smoke(), and the
 * cpu_baseline leg of bench.py).  The product package never links or calls it.
 *
 * Formulation.  The reference builds, per neuron, a queue of columns
 * (salt_core/connectivity/{fc,conv}.py), looks up decay codes
 * (salt_core/quant/codes.py:87-105) and scans every column with process_event
 * (salt_core/quant/scan.py:22-52, 97-132), then extracts the spike stream
 * (salt_core/stream.py:24-100).  This file restates the same computation event by
 * event: each neuron keeps its register and the time of its last queue column, and
 * the columns the reference adds that carry no event (FC pads, the conv catch-up
 * column and the identity columns after it) are replayed explicitly, so that the
 * final register, the min/max of the pre-write-back value, the spike stream and its
 * truncation at capacity all come out as the queue formulation gives them.
 *
 * Integer conventions: int32 two's complement with wrap-around (as XLA computes
 * int32), arithmetic right shift of negative values (gcc), float32 times.
 */
#include "salt_oracle.h"

#include <limits.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define PAD_TIME 1e12f /* salt_core/stream.py:13 */

/* ---------------------------------------------------------------- fixed point */

/* salt_core/quant/fixed_point.py:32-44: add half (ROUND) then arithmetic shift. */
static inline int32_t round_shift_i(int64_t x, int32_t shift_bits, int32_t round_mode) {
    if (shift_bits == 0) return (int32_t)x;
    if (round_mode == 0) x += (int64_t)1 << (shift_bits - 1);
    return (int32_t)(x >> shift_bits);
}
int32_t oracle_round_shift(int64_t x, int32_t shift_bits, int32_t round_mode) {
    return round_shift_i(x, shift_bits, round_mode);
}

/* salt_core/quant/fixed_point.py:47-65.  The reference splits v into hi/lo halves so
 * that no product leaves int32; the result is, bit for bit, round_shift(a*v) on the
 * exact product (proved in the reference's docs and tested there against Python
 * big integers, test_fixed_point.py:101-122).  The oracle computes that exact
 * product in 64 bits instead -- a different mechanism from the GPU kernel's split. */
static inline int32_t wide_mul_shift_i(int32_t a, int32_t v, int32_t shift_bits,
                                       int32_t round_mode) {
    return round_shift_i((int64_t)a * (int64_t)v, shift_bits, round_mode);
}
int32_t oracle_wide_mul_shift(int32_t a, int32_t v, int32_t shift_bits, int32_t round_mode) {
    return wide_mul_shift_i(a, v, shift_bits, round_mode);
}

/* salt_core/quant/fixed_point.py:68-90: write back into a total_bits-wide signed
 * register, wrap (two's complement) or saturate; flag values out of range. */
static inline int32_t fit_to_bits_i(int32_t x, int32_t total_bits, int32_t overflow_mode,
                                    int32_t* overflowed) {
    int64_t half = (int64_t)1 << (total_bits - 1);
    int64_t xv = x;
    if (overflowed) *overflowed = (xv < -half) || (xv >= half);
    if (overflow_mode == 1) {
        if (xv < -half) return (int32_t)(-half);
        if (xv >= half) return (int32_t)(half - 1);
        return x;
    }
    int64_t modulus = (int64_t)1 << total_bits;
    int64_t masked = xv & (modulus - 1);
    return (int32_t)(masked >= half ? masked - modulus : masked);
}
int32_t oracle_fit_to_bits(int32_t x, int32_t total_bits, int32_t overflow_mode,
                           int32_t* overflowed) {
    return fit_to_bits_i(x, total_bits, overflow_mode, overflowed);
}

/* salt_core/quant/codes.py:87-105: dt == 0 -> identity; 1 <= dt <= n -> table[dt-1];
 * dt > n -> 0.  dt is a float32 holding integer ms; XLA converts it to int32 with
 * saturation, then clips the gather index to [0, n-1]. */
static inline int32_t decay_lookup_i(float delta_t, const int32_t* table, int32_t n_table,
                                     int32_t* is_identity) {
    int64_t d;
    if (delta_t >= 2147483647.0f) d = INT32_MAX;
    else if (delta_t <= -2147483648.0f) d = INT32_MIN;
    else d = (int64_t)delta_t; /* truncation toward zero, as astype(int32) */
    if (is_identity) *is_identity = (d == 0);
    int64_t idx = d - 1;
    if (idx < 0) idx = 0;
    if (idx > n_table - 1) idx = n_table - 1;
    int32_t gathered = table[idx];
    return d > n_table ? 0 : gathered;
}
int32_t oracle_decay_lookup(float delta_t, const int32_t* table, int32_t n_table,
                            int32_t* is_identity) {
    return decay_lookup_i(delta_t, table, n_table, is_identity);
}

/* salt_core/quant/scan.py:22-52. */
static inline int32_t process_event_i(int32_t v0, int32_t a_int, int32_t is_identity, int32_t q,
                                      int32_t has_vth, int32_t v_th, int32_t f_a, int32_t f_V,
                                      int32_t i_V, int32_t round_mode, int32_t overflow_mode,
                                      int32_t* spiked, int32_t* overflowed,
                                      int32_t* v_unfitted) {
    int32_t decayed = is_identity ? v0 : wide_mul_shift_i(a_int, v0, f_a, round_mode);
    /* decayed + q * (1 << f_V) in wrapping int32 */
    int32_t unfitted = (int32_t)((uint32_t)decayed + ((uint32_t)q << f_V));
    int32_t ovf = 0;
    int32_t fitted = fit_to_bits_i(unfitted, i_V + f_V, overflow_mode, &ovf);
    int32_t sp = has_vth ? (fitted >= v_th) : 0;
    if (spiked) *spiked = sp;
    if (overflowed) *overflowed = ovf;
    if (v_unfitted) *v_unfitted = unfitted;
    return sp ? 0 : fitted;
}
int32_t oracle_process_event(int32_t v0, int32_t a_int, int32_t is_identity, int32_t q,
                             int32_t has_vth, int32_t v_th, int32_t f_a, int32_t f_V,
                             int32_t i_V, int32_t round_mode, int32_t overflow_mode,
                             int32_t* spiked, int32_t* overflowed, int32_t* v_unfitted) {
    return process_event_i(v0, a_int, is_identity, q, has_vth, v_th, f_a, f_V, i_V, round_mode,
                           overflow_mode, spiked, overflowed, v_unfitted);
}

/* ---------------------------------------------------------------- spike buffers */

typedef struct {
    int32_t* j;      /* global event index of the triggering column (sort key) */
    int32_t* neuron; /* neuron id */
    int64_t n, capacity;
} spike_buf;

static void sb_push(spike_buf* b, int32_t j, int32_t neuron) {
    if (b->n == b->capacity) {
        b->capacity = b->capacity ? b->capacity * 2 : 4096;
        b->j = (int32_t*)realloc(b->j, (size_t)b->capacity * sizeof(int32_t));
        b->neuron = (int32_t*)realloc(b->neuron, (size_t)b->capacity * sizeof(int32_t));
    }
    b->j[b->n] = j;
    b->neuron[b->n] = neuron;
    b->n++;
}

static inline uint64_t mix64(uint64_t z);

/* One kept entry of the output stream: written where asked, and mixed into the
 * order-sensitive hash of oracle_stream_hash (entry index i, time bits, source). */
static inline void put_entry(int64_t i, float t, int32_t s, float* out_times, int32_t* out_src,
                             uint64_t* hash_acc) {
    if (out_times) out_times[i] = t;
    if (out_src) out_src[i] = s;
    if (hash_acc) {
        uint32_t tb;
        memcpy(&tb, &t, 4);
        *hash_acc += mix64(mix64((uint64_t)i) ^ (((uint64_t)tb << 32) | (uint32_t)s));
    }
}

/*
 * salt_core/stream.py:24-64.  The reference takes the first `cap` spikes of
 * nonzero(spike_mask) -- neuron-major, then queue column -- and sorts them stably by
 * global event index.  `spikes` arrive here in (j, neuron) order with, per neuron,
 * increasing column; keeping the ones whose neuron-major rank is below cap and
 * leaving the (j, neuron) order as it is gives the same stream.
 */
static void emit_stream(const spike_buf* sb, int32_t n_neurons, int32_t cap,
                        const float* times, int32_t L, float* out_times, int32_t* out_src,
                        int32_t* out_n, int32_t* scratch_counts, uint64_t* out_hash) {
    int64_t total = sb->n;
    *out_n = (int32_t)total;
    uint64_t acc = 0;
    uint64_t* hacc = out_hash ? &acc : NULL;
    if (!out_times && !out_src && !out_hash) return;
    int64_t written = 0;
    if (total <= cap) {
        for (int64_t i = 0; i < total; i++) {
            int32_t j = sb->j[i];
            int32_t jj = j < L ? j : L - 1; /* stream.py:37-38 clamps the pad index */
            put_entry(written, times[jj], sb->neuron[i], out_times, out_src, hacc);
            written++;
        }
    } else {
        /* neuron-major rank: start offset of each neuron + rank within the neuron */
        memset(scratch_counts, 0, sizeof(int32_t) * (size_t)n_neurons);
        for (int64_t i = 0; i < total; i++) scratch_counts[sb->neuron[i]]++;
        int64_t acc = 0;
        for (int32_t n = 0; n < n_neurons; n++) {
            int32_t c = scratch_counts[n];
            scratch_counts[n] = (int32_t)(acc > INT32_MAX ? INT32_MAX : acc);
            acc += c;
        }
        for (int64_t i = 0; i < total && written < cap; i++) {
            int32_t n = sb->neuron[i];
            int64_t rank = scratch_counts[n]++;
            if (rank < cap) {
                int32_t j = sb->j[i];
                int32_t jj = j < L ? j : L - 1;
                put_entry(written, times[jj], n, out_times, out_src, hacc);
                written++;
            }
        }
    }
    for (int64_t i = written; i < cap; i++) {
        if (out_times) out_times[i] = PAD_TIME;
        if (out_src) out_src[i] = 0; /* nonzero(..., fill_value=0), stream.py:60 */
    }
    if (out_hash) *out_hash = mix64(acc + (uint64_t)(uint32_t)total * 0x2545F4914F6CDD1DULL);
}

/* ---------------------------------------------------------------- layer */

typedef struct {
    int32_t f_a, f_V, i_V, rm, om;
    int32_t vth_kind;
    const int32_t* vth;
    int32_t can_fire_on_identity; /* some threshold <= 0: identity columns may fire */
} step_cfg;

static inline int32_t vth_of(const step_cfg* c, int32_t neuron) {
    return c->vth_kind == ORACLE_VTH_SCALAR ? c->vth[0] : c->vth[neuron];
}

static inline void step(const step_cfg* c, int32_t* V, int32_t* vmin, int32_t* vmax,
                        int32_t neuron, int32_t a, int32_t ident, int32_t q, int32_t j,
                        spike_buf* sb) {
    int32_t sp, ovf, u;
    int32_t has = c->vth_kind != ORACLE_VTH_NONE;
    V[neuron] = process_event_i(V[neuron], a, ident, q, has, has ? vth_of(c, neuron) : 0,
                                c->f_a, c->f_V, c->i_V, c->rm, c->om, &sp, &ovf, &u);
    if (u < vmin[neuron]) vmin[neuron] = u;
    if (u > vmax[neuron]) vmax[neuron] = u;
    if (sp) sb_push(sb, j, neuron);
}

/* Python's floor division for the candidate formulas of connectivity/conv.py:15-29. */
static inline int32_t floordiv(int32_t a, int32_t b) {
    int32_t q = a / b;
    if ((a % b != 0) && ((a < 0) != (b < 0))) q--;
    return q;
}

/* FC layer for one stream: connectivity/fc.py:20-33, 54-61; layers/fc.py:84-124. */
static void fc_stream(const oracle_geom* g, const oracle_qparams* p, const step_cfg* c,
                      int32_t L, const float* t, const int32_t* src, int32_t n_real,
                      int32_t* V, int32_t* vmin, int32_t* vmax, spike_buf* sb) {
    int32_t N = g->n_out;
    int32_t n_eff = n_real < 0 ? 0 : (n_real < L ? n_real : L);
    float t_prev = 0.0f; /* the first event is compared with t = 0 (fc.py:30) */
    for (int32_t j = 0; j < n_eff; j++) {
        float dt = t[j] - t_prev; /* float32 difference, fc.py:28-30 */
        int32_t ident;
        int32_t a = decay_lookup_i(dt, p->table, p->n_table, &ident);
        int32_t s = src[j];
        for (int32_t i = 0; i < N; i++)
            step(c, V, vmin, vmax, i, a, ident, p->q[(int64_t)i * g->n_in + s], j, sb);
        t_prev = t[j];
    }
    /* Pad columns: dt = 0 (identity), code 0 (fc.py:32, :60-61). */
    if (n_eff < L) {
        if (c->can_fire_on_identity) {
            for (int32_t j = n_eff; j < L; j++)
                for (int32_t i = 0; i < N; i++) step(c, V, vmin, vmax, i, 0, 1, 0, j, sb);
        } else {
            for (int32_t i = 0; i < N; i++) { /* U = V on every pad column, no fire */
                if (V[i] < vmin[i]) vmin[i] = V[i];
                if (V[i] > vmax[i]) vmax[i] = V[i];
            }
        }
    }
}

/* Conv layer for one stream: connectivity/conv.py:15-225; layers/conv.py:124-175.
 * t_last and the candidate count are per spatial position (conv.py:46-54). */
static void conv_stream(const oracle_geom* g, const oracle_qparams* p, const step_cfg* c,
                        int32_t L, const float* t, const int32_t* src, int32_t n_real,
                        int32_t* V, int32_t* vmin, int32_t* vmax, spike_buf* sb,
                        float* t_last, int32_t* cnt, int32_t* act_a, int32_t* act_id,
                        int32_t* act_pos, int32_t* act_ky, int32_t* act_kx,
                        int32_t* needed) {
    const int32_t K = g->k, S = g->s, P = g->p;
    const int32_t H = (g->h_in + 2 * P - K) / S + 1, W = (g->w_in + 2 * P - K) / S + 1;
    const int32_t HW = H * W, hw_in = g->h_in * g->w_in, OC = g->oc;
    const int32_t ncand = (K - 1) / S + 1;
    const int32_t mql = g->max_queue_len;
    const int32_t n_eff = n_real < 0 ? 0 : (n_real < L ? n_real : L);
    for (int32_t i = 0; i < HW; i++) { t_last[i] = 0.0f; cnt[i] = 0; }

    for (int32_t j = 0; j < n_eff; j++) {
        int32_t s = src[j];
        int32_t ch = s / hw_in, rem = s % hw_in, y = rem / g->w_in, x = rem % g->w_in;
        int32_t oy0 = floordiv(y + P - K + 1 + S - 1, S), oy_hi = floordiv(y + P, S);
        int32_t ox0 = floordiv(x + P - K + 1 + S - 1, S), ox_hi = floordiv(x + P, S);
        int32_t n_act = 0;
        for (int32_t ry = 0; ry < ncand; ry++) {
            int32_t oy = oy0 + ry;
            if (oy > oy_hi || oy < 0 || oy >= H) continue;
            for (int32_t rx = 0; rx < ncand; rx++) {
                int32_t ox = ox0 + rx;
                if (ox > ox_hi || ox < 0 || ox >= W) continue;
                int32_t pos = oy * W + ox;
                int32_t before = cnt[pos]++;
                if (before >= mql) continue; /* dropped: the queue is full (conv.py:143-151) */
                float dt = t[j] - t_last[pos]; /* real column: gap to previous (conv.py:180) */
                act_a[n_act] = decay_lookup_i(dt, p->table, p->n_table, &act_id[n_act]);
                act_pos[n_act] = pos;
                act_ky[n_act] = y - oy * S + P;
                act_kx[n_act] = x - ox * S + P;
                n_act++;
            }
        }
        /* Neuron id oc*HW + pos; oc-major then ascending pos is ascending id, which is
         * the order stream.py:29-30 puts simultaneous spikes in. */
        for (int32_t oc = 0; oc < OC; oc++) {
            const int32_t* qo = p->q + (int64_t)oc * g->ic * K * K + (int64_t)ch * K * K;
            for (int32_t a = 0; a < n_act; a++)
                step(c, V, vmin, vmax, oc * HW + act_pos[a], act_a[a], act_id[a],
                     qo[act_ky[a] * K + act_kx[a]], j, sb);
        }
        for (int32_t a = 0; a < n_act; a++) t_last[act_pos[a]] = t[j];
    }

    /* Catch-up column (col == n_real_pos) decays to the last real input time T, then
     * identity columns up to max_queue_len (conv.py:163-186).  Their spikes, if any,
     * map to the sentinel global index L (conv.py:149) and sort after every real one. */
    int32_t maxcnt = 0;
    for (int32_t pos = 0; pos < HW; pos++) if (cnt[pos] > maxcnt) maxcnt = cnt[pos];
    *needed = maxcnt + 1; /* layers/conv.py:137-139 */
    float T = n_eff > 0 ? t[n_eff - 1] : (L > 0 ? t[L - 1] : 0.0f);
    /* The catch-up and identity columns are applied neuron by neuron, so their spikes
     * are pushed per neuron in column order; they all share key L. */
    for (int32_t oc = 0; oc < OC; oc++) {
        for (int32_t pos = 0; pos < HW; pos++) {
            if (cnt[pos] >= mql) continue;
            int32_t neuron = oc * HW + pos;
            /* An empty position's catch-up reads t_gathered = T, so its dt is 0. */
            float dt = cnt[pos] > 0 ? T - t_last[pos] : 0.0f;
            int32_t ident;
            int32_t a = decay_lookup_i(dt, p->table, p->n_table, &ident);
            step(c, V, vmin, vmax, neuron, a, ident, 0, L, sb);
            int32_t n_identity = mql - cnt[pos] - 1;
            if (n_identity > 0) {
                if (c->can_fire_on_identity) {
                    for (int32_t k = 0; k < n_identity; k++)
                        step(c, V, vmin, vmax, neuron, 0, 1, 0, L, sb);
                } else {
                    if (V[neuron] < vmin[neuron]) vmin[neuron] = V[neuron];
                    if (V[neuron] > vmax[neuron]) vmax[neuron] = V[neuron];
                }
            }
        }
    }
}

static int layer_forward_impl(const oracle_geom* g, const oracle_qparams* prm, int32_t B,
                              int32_t L, const float* times, const int32_t* src,
                              const int32_t* n_real, int32_t cap, float* out_times,
                              int32_t* out_src, int32_t* out_n, uint64_t* out_hash,
                              int32_t* v_final, int32_t* v_min, int32_t* v_max,
                              int32_t* needed_queue, int32_t nthreads) {
    if (!g || !prm || B < 0 || L < 0 || cap < 0 || !out_n) return -1;
    if (prm->n_table < 1 || prm->f_a < 0 || prm->f_a > 15 || prm->f_V < 0 ||
        prm->i_V + prm->f_V < 1 || prm->i_V + prm->f_V > 30)
        return -1;
    int32_t N, HW = 1;
    if (g->kind == ORACLE_FC) {
        N = g->n_out;
    } else if (g->kind == ORACLE_CONV) {
        if (g->k < 1 || g->s < 1 || g->p < 0 || g->max_queue_len < 1) return -1;
        int32_t H = (g->h_in + 2 * g->p - g->k) / g->s + 1;
        int32_t W = (g->w_in + 2 * g->p - g->k) / g->s + 1;
        if (H < 1 || W < 1) return -1;
        HW = H * W;
        N = g->oc * HW;
    } else {
        return -1;
    }
    step_cfg c = {prm->f_a, prm->f_V, prm->i_V, prm->round_mode, prm->overflow_mode,
                  prm->v_th_kind, prm->v_th, 0};
    if (c.vth_kind == ORACLE_VTH_SCALAR) c.can_fire_on_identity = prm->v_th[0] <= 0;
    if (c.vth_kind == ORACLE_VTH_PER_NEURON)
        for (int32_t i = 0; i < N; i++) if (prm->v_th[i] <= 0) c.can_fire_on_identity = 1;

#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        spike_buf sb = {0};
        int32_t* Vs = (int32_t*)malloc(sizeof(int32_t) * (size_t)N * 3);
        int32_t* counts = (int32_t*)malloc(sizeof(int32_t) * (size_t)N);
        float* t_last = (float*)malloc(sizeof(float) * (size_t)HW);
        int32_t* cnt = (int32_t*)malloc(sizeof(int32_t) * (size_t)HW);
        int32_t nc = g->kind == ORACLE_CONV ? ((g->k - 1) / g->s + 1) : 1;
        int32_t* act = (int32_t*)malloc(sizeof(int32_t) * (size_t)nc * nc * 5);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int32_t b = 0; b < B; b++) {
            int32_t *V = Vs, *vmn = Vs + N, *vmx = Vs + 2 * (size_t)N;
            memset(Vs, 0, sizeof(int32_t) * (size_t)N * 3);
            sb.n = 0;
            const float* tb = times + (int64_t)b * L;
            const int32_t* sbp = src + (int64_t)b * L;
            int32_t needed = 0;
            if (g->kind == ORACLE_FC)
                fc_stream(g, prm, &c, L, tb, sbp, n_real[b], V, vmn, vmx, &sb);
            else
                conv_stream(g, prm, &c, L, tb, sbp, n_real[b], V, vmn, vmx, &sb, t_last, cnt,
                            act, act + nc * nc, act + 2 * nc * nc, act + 3 * nc * nc,
                            act + 4 * nc * nc, &needed);
            /* Real spikes were pushed in (j, neuron) order and catch-up/identity
             * spikes (key L) after them in neuron order: the buffer is already in
             * the stable key order of stream.py:40. */
            emit_stream(&sb, N, cap, tb, L, out_times ? out_times + (int64_t)b * cap : NULL,
                        out_src ? out_src + (int64_t)b * cap : NULL, &out_n[b], counts,
                        out_hash ? &out_hash[b] : NULL);
            if (v_final) memcpy(v_final + (int64_t)b * N, V, sizeof(int32_t) * (size_t)N);
            if (v_min) memcpy(v_min + (int64_t)b * N, vmn, sizeof(int32_t) * (size_t)N);
            if (v_max) memcpy(v_max + (int64_t)b * N, vmx, sizeof(int32_t) * (size_t)N);
            if (needed_queue) needed_queue[b] = g->kind == ORACLE_CONV ? needed : 0;
        }
        free(sb.j);
        free(sb.neuron);
        free(Vs);
        free(counts);
        free(t_last);
        free(cnt);
        free(act);
    }
    return 0;
}

int oracle_layer_forward(const oracle_geom* g, const oracle_qparams* prm, int32_t B,
                         int32_t L, const float* times, const int32_t* src,
                         const int32_t* n_real, int32_t cap, float* out_times,
                         int32_t* out_src, int32_t* out_n, int32_t* v_final,
                         int32_t* v_min, int32_t* v_max, int32_t* needed_queue,
                         int32_t nthreads) {
    return layer_forward_impl(g, prm, B, L, times, src, n_real, cap, out_times, out_src, out_n,
                              NULL, v_final, v_min, v_max, needed_queue, nthreads);
}

int oracle_layer_forward_hashed(const oracle_geom* g, const oracle_qparams* prm, int32_t B,
                                int32_t L, const float* times, const int32_t* src,
                                const int32_t* n_real, int32_t cap, int32_t* out_n,
                                uint64_t* out_hash, int32_t* v_final, int32_t* v_min,
                                int32_t* v_max, int32_t* needed_queue, int32_t nthreads) {
    if (!out_hash) return -1;
    return layer_forward_impl(g, prm, B, L, times, src, n_real, cap, NULL, NULL, out_n,
                              out_hash, v_final, v_min, v_max, needed_queue, nthreads);
}

/* ---------------------------------------------------------------- stream hash */

static inline uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

uint64_t oracle_stream_hash(const float* times, const int32_t* src, int32_t n, int32_t cap) {
    int32_t m = n < cap ? n : cap;
    uint64_t acc = 0;
    for (int32_t i = 0; i < m; i++) {
        uint32_t tb;
        memcpy(&tb, &times[i], 4);
        uint64_t key = ((uint64_t)tb << 32) | (uint32_t)src[i];
        acc += mix64(mix64((uint64_t)i) ^ key);
    }
    return mix64(acc + (uint64_t)(uint32_t)n * 0x2545F4914F6CDD1DULL);
}
