/*
 * CPU oracle for the integer event-by-event forward pass of salt_core/quant.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP path is
 * compared against (tests/, __graft_entry__.smoke(), and the cpu_baseline leg of
 * bench.py).  Nothing in the product package may link, load or call it.
 *
 * It is an event-driven restatement of the reference's queue formulation: every
 * function cites the reference file:line whose behaviour it restates.  The
 * reference itself (Python on JAX) cannot run in this image, so the oracle is
 * pinned by the reference's own known-answer tests (the JSON fixtures in tests/golden), by a
 * second, literal NumPy restatement of the queue formulation (oracle/queue_ref.py),
 * and by closed forms (exact 64-bit arithmetic for the shift-rounded multiply).
 */
#ifndef SALT_ORACLE_H
#define SALT_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Layer kinds. */
#define ORACLE_FC 0
#define ORACLE_CONV 1

/* v_th kinds: no threshold (never fires), one scalar, one value per neuron. */
#define ORACLE_VTH_NONE 0
#define ORACLE_VTH_SCALAR 1
#define ORACLE_VTH_PER_NEURON 2

typedef struct {
    int32_t kind;          /* ORACLE_FC or ORACLE_CONV                                   */
    int32_t n_in, n_out;   /* FC geometry (n_out = neurons)                               */
    int32_t ic, h_in, w_in, oc, k, s, p; /* conv geometry, salt_core/layers/conv.py:30-39 */
    int32_t max_queue_len; /* conv per-position queue capacity, layers/conv.py:49         */
} oracle_geom;

typedef struct {
    const int32_t* q;      /* weight codes as int32, reference layout: FC (n_out, n_in),
                              conv (oc, ic, k, k) -- quant/params.py:11-12             */
    const int32_t* table;  /* decay_table_int, length n_table (dt = 1 .. n_table)         */
    int32_t n_table;
    const int32_t* v_th;   /* see v_th_kind                                              */
    int32_t v_th_kind;
    int32_t f_a, f_V, i_V;
    int32_t round_mode;    /* 0 = round, 1 = truncate  (fixed_point.py:20-23)             */
    int32_t overflow_mode; /* 0 = wrap,  1 = saturate  (fixed_point.py:26-29)             */
} oracle_qparams;

/* Scalar primitives, exported so that the tests can pin them one by one. */
int32_t oracle_round_shift(int64_t x, int32_t shift_bits, int32_t round_mode);
int32_t oracle_wide_mul_shift(int32_t a, int32_t v, int32_t shift_bits, int32_t round_mode);
int32_t oracle_fit_to_bits(int32_t x, int32_t total_bits, int32_t overflow_mode,
                           int32_t* overflowed);
int32_t oracle_decay_lookup(float delta_t, const int32_t* table, int32_t n_table,
                            int32_t* is_identity);
/* One process_event step; returns the new register value. */
int32_t oracle_process_event(int32_t v0, int32_t a_int, int32_t is_identity, int32_t q,
                             int32_t has_vth, int32_t v_th, int32_t f_a, int32_t f_V,
                             int32_t i_V, int32_t round_mode, int32_t overflow_mode,
                             int32_t* spiked, int32_t* overflowed, int32_t* v_unfitted);

/*
 * One layer over a batch of B padded streams of length L.
 *   times[B*L] float32 ms, src[B*L], n_real[B]   (stream.py:16-21)
 *   cap: output stream length (max_out_spikes).
 * Outputs (any may be NULL except out_n):
 *   out_times/out_src [B*cap]: the reference EventStream (pads: 1e12, 0)
 *   out_n[B]: total spike count (may exceed cap)
 *   v_final/v_min/v_max [B*N]: register after the layer; min/max of the value before
 *     write-back over every queue column and the initial 0 (quant/scan.py:116-117)
 *   needed_queue[B]: conv only, max per-position candidate count + 1 (layers/conv.py:139)
 * nthreads <= 0 uses all OpenMP threads.  Returns 0, or -1 on invalid arguments.
 */
int oracle_layer_forward(const oracle_geom* g, const oracle_qparams* prm, int32_t B,
                         int32_t L, const float* times, const int32_t* src,
                         const int32_t* n_real, int32_t cap, float* out_times,
                         int32_t* out_src, int32_t* out_n, int32_t* v_final,
                         int32_t* v_min, int32_t* v_max, int32_t* needed_queue,
                         int32_t nthreads);

/* oracle_layer_forward without the output stream: per stream, its spike count and the
 * hash oracle_stream_hash would give of the stream it writes (no B*cap buffers, for
 * streams of millions of spikes).  v_final/v_min/v_max/needed_queue as above. */
int oracle_layer_forward_hashed(const oracle_geom* g, const oracle_qparams* prm, int32_t B,
                                int32_t L, const float* times, const int32_t* src,
                                const int32_t* n_real, int32_t cap, int32_t* out_n,
                                uint64_t* out_hash, int32_t* v_final, int32_t* v_min,
                                int32_t* v_max, int32_t* needed_queue, int32_t nthreads);

/* Order-sensitive 64-bit hash of one output stream, for streams too large to copy
 * back.  Each entry i < min(n, cap) contributes mix64(mix64(i) ^ (time_bits << 32 | src));
 * the contributions are summed mod 2^64 (so a GPU can reduce them in any order) and
 * the sum is finalised with n.  The entry index inside the mix makes it order-sensitive. */
uint64_t oracle_stream_hash(const float* times, const int32_t* src, int32_t n, int32_t cap);

#ifdef __cplusplus
}
#endif
#endif
