/*
 * libsalt_hip.so -- C-ABI of the MI355X (gfx950) integer event-by-event forward pass.
 *
 * This is the drop-in boundary for the hot path of salt_core/quant.  In the reference the
 * path is reached through the backend seam
 *     QuantBackend.scan(layer, structure, params, event_gain, trace)   salt_core/quant/backend.py:31-53
 * called by ConvLayer.forward / FCLayer.forward (salt_core/layers/conv.py:124-149,
 * salt_core/layers/fc.py:84-101), followed by the stream extraction of
 * salt_core/stream.py:67-100.  An event-driven kernel subsumes queue construction
 * (salt_core/connectivity/{fc,conv}.py), the scan (salt_core/quant/scan.py:97-132) and the
 * extraction, so one entry point here replaces that whole per-layer chain:
 * events in -> spike stream + registers + diagnostics out.
 *
 * Conventions
 *  - Every pointer named d_* is a device pointer (hipMalloc'ed or from a framework
 *    allocator); h_* pointers are host pointers.  No torch or framework types appear.
 *  - Calls are asynchronous on `stream` (a hipStream_t; NULL = default stream) unless
 *    stated.  The library keeps no reference to any buffer after a call returns.
 *  - Return value: 0 = OK; <0 = error: -1 invalid argument, -2 HIP error,
 *    -3 unsupported geometry.  salt_last_error() describes the last nonzero return of
 *    the calling thread.  Capacity overflow (fits == False in the reference) is not an
 *    error: it shows in the outputs (d_n > cap, stats needed > max_queue_len).
 *  - Weight codes are int8/int16/int32; times are float32 holding integer milliseconds
 *    (salt_core/stream.py:16-21 keeps times as float32); registers are int32.
 */
#ifndef SALT_HIP_H
#define SALT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SALT_ABI_VERSION 1

#define SALT_LAYER_FC 0
#define SALT_LAYER_CONV 1

#define SALT_VTH_NONE 0        /* v_th_int = None: never fires (quant/params.py:14-15)   */
#define SALT_VTH_SCALAR 1      /* one threshold for every neuron                         */
#define SALT_VTH_PER_CHANNEL 2 /* conv: one per output channel; FC: one per neuron       */
#define SALT_VTH_PER_NEURON 3  /* one per neuron, neuron = oc*H*W + y*W + x              */

#define SALT_ROUND 0           /* fixed_point.py:20-23 */
#define SALT_TRUNCATE 1
#define SALT_WRAP 0            /* fixed_point.py:26-29 */
#define SALT_SATURATE 1

/* Layer geometry and capacities.  Mirrors ConvLayer (salt_core/layers/conv.py:30-53) and
 * FCLayer (salt_core/layers/fc.py:23-38); the float-training fields are not needed. */
typedef struct {
    int32_t kind;            /* SALT_LAYER_FC or SALT_LAYER_CONV                       */
    int32_t n_in, n_out;     /* FC                                                     */
    int32_t ic, h_in, w_in;  /* conv input plane                                       */
    int32_t oc, k, s, p;     /* conv output channels, kernel, stride, padding          */
    int32_t max_queue_len;   /* conv capacity (layers/conv.py:49)                      */
    int32_t max_out_spikes;  /* output stream length per stream (layers/conv.py:50)    */
} salt_layer_desc;

/* Quantized parameters.  Mirrors QuantizedLayerParams (salt_core/quant/params.py:9-21)
 * plus QuantBackend.round_mode (salt_core/quant/backend.py:24-29). */
typedef struct {
    const void* d_q;          /* weight codes: conv (oc, ic, k, k) as in the reference;
                                 FC transposed to (n_in, n_out) -- see salt_fc_transpose */
    int32_t q_bits;           /* 8, 16 or 32                                             */
    const int32_t* d_decay_table; /* decay_table_int, dt = 1 .. n_table                  */
    int32_t n_table;          /* >= 1                                                    */
    const int32_t* d_v_th;    /* per-channel / per-neuron thresholds, or NULL            */
    int32_t v_th_kind;        /* SALT_VTH_*                                              */
    int32_t v_th_scalar;      /* used when v_th_kind == SALT_VTH_SCALAR                  */
    int32_t f_a, f_V, i_V;    /* 0 <= f_a <= 15, 1 <= i_V + f_V <= 30                    */
    int32_t round_mode;       /* SALT_ROUND / SALT_TRUNCATE                              */
    int32_t overflow_mode;    /* SALT_WRAP / SALT_SATURATE                               */
} salt_qparams;

/* A batch of padded event streams (EventStream, salt_core/stream.py:16-21, batched). */
typedef struct {
    int32_t B, L;
    const float* d_times;     /* [B*L]; real part non-decreasing integer ms           */
    const int32_t* d_src;     /* [B*L]; source neuron id, flat over the input shape   */
    const int32_t* d_n_real;  /* [B]; may exceed L (all L entries are then real)      */
} salt_events_in;

typedef struct {
    int32_t cap;              /* == max_out_spikes                                    */
    float* d_times;           /* [B*cap] spike time = time of the triggering event    */
    int32_t* d_src;           /* [B*cap] neuron id                                    */
    int32_t* d_n;             /* [B] total spike count, may exceed cap               */
    int32_t fill_pads;        /* nonzero: entries n..cap-1 get time 1e12, src 0
                                 (stream.py:13, :60), as the reference's stream has   */
} salt_events_out;

/* Per-layer results.  Mirrors QuantLayerResult (salt_core/quant/scan.py:55-62) in
 * event-driven form: the (n, queue_len) masks are replaced by the spike stream, and the
 * per-step overflow flags by their per-neuron / per-stream reductions. */
typedef struct {
    int32_t* d_v_final;       /* [B*N] register after the layer (NULL: not written)   */
    int32_t* d_v_min;         /* [B*N] v_unfitted_min per neuron, or NULL             */
    int32_t* d_v_max;         /* [B*N] v_unfitted_max per neuron, or NULL             */
    int32_t* d_stats;         /* [B*4] per stream: min over neurons of v_unfitted_min,
                                 max of v_unfitted_max, needed max_queue_len (conv;
                                 layers/conv.py:137-139; 0 for FC), overflowed (0/1)  */
} salt_layer_result;

int32_t salt_version(void);
const char* salt_last_error(void);

/* Device memory helpers so that a caller needs no framework (plain hipMalloc/hipFree). */
int32_t salt_malloc(void** d_ptr, size_t bytes);
int32_t salt_free(void* d_ptr);
int32_t salt_memcpy_h2d(void* d_dst, const void* h_src, size_t bytes, void* stream);
int32_t salt_memcpy_d2h(void* h_dst, const void* d_src, size_t bytes, void* stream);
int32_t salt_stream_sync(void* stream);

/* Transpose FC weight codes from the reference layout (n_out, n_in)
 * (FCLayer.weight_shape, salt_core/layers/fc.py:58-60) to the (n_in, n_out) layout the
 * FC kernels read;
 * replaces the per-event gather q[:, src] of salt_core/connectivity/fc.py:54-61. */
int32_t salt_fc_transpose(const void* d_q_ref, void* d_q_t, int32_t n_out, int32_t n_in,
                          int32_t q_bits, void* stream);

/* Bytes of device workspace salt_layer_forward needs for this layer and batch. */
int32_t salt_layer_workspace_size(const salt_layer_desc* desc, const salt_qparams* prm,
                                  int32_t B, int32_t L, int32_t want_neuron_extremes,
                                  size_t* bytes);

/*
 * One layer over a batch: replaces QuantBackend.scan + stream extraction for
 * ConvLayer.forward / FCLayer.forward (salt_core/layers/conv.py:124-149,
 * salt_core/layers/fc.py:84-101; salt_core/quant/backend.py:31-53;
 * salt_core/stream.py:67-100).  Host-side argument checks mirror the reference's
 * ValueErrors (fixed_point.py:57-60, :79-82) and reject a scalar threshold <= 0.
 * Preconditions on device data, which the caller checks (the Python host layer does):
 * thresholds > 0, source ids in range, real times non-decreasing integers, decay codes
 * in [0, 2^f_a).  Violating them gives wrong values but never an out-of-bounds access.
 * When result->d_v_min/d_v_max are non-NULL the per-neuron extremes are computed
 * (slower); the per-stream stats are always computed.
 * d_workspace must hold salt_layer_workspace_size() bytes.
 * A stream that produced more than cap spikes gets d_n > cap and only the first cap
 * spikes in (event, neuron) order; the reference instead keeps the first cap in
 * (neuron, column) order (salt_core/stream.py:60), which a caller reproduces by
 * re-running with a larger cap and selecting.
 */
int32_t salt_layer_forward(const salt_layer_desc* desc, const salt_qparams* prm,
                           const salt_events_in* in, const salt_events_out* out,
                           const salt_layer_result* result, void* d_workspace,
                           size_t workspace_bytes, void* stream);

/* Bytes of device workspace salt_network_forward needs: the largest of the layers'
 * salt_layer_workspace_size() (the layers run one after the other on one stream, so they
 * share it), layer i > 0 reading a stream of L = descs[i-1].max_out_spikes entries. */
int32_t salt_network_workspace_size(int32_t n_layers, const salt_layer_desc* descs,
                                    const salt_qparams* prms, int32_t B, int32_t L,
                                    int32_t want_neuron_extremes, size_t* bytes);

/*
 * A whole network over a batch in one call: replaces run_network's layer loop
 * (salt_core/network.py:93-122, each layer's output stream feeding the next).  Layer i
 * runs as salt_layer_forward with input outs[i-1] (L = its cap, n_real = its d_n, of
 * which the first min(d_n, cap) entries are read), all on `stream` with no host
 * synchronisation.  descs/prms/outs/results: arrays of n_layers entries, as for
 * salt_layer_forward; every results[i] gives both or neither of d_v_min/d_v_max.  All
 * arguments are checked before the first launch.  A stream whose layer i exceeded its
 * cap feeds layer i+1 with the first cap spikes in (event, neuron) order (fits = false:
 * the reference's truncation keeps a different subset, salt_core/stream.py:60).
 */
int32_t salt_network_forward(int32_t n_layers, const salt_layer_desc* descs,
                             const salt_qparams* prms, const salt_events_in* in,
                             const salt_events_out* outs, const salt_layer_result* results,
                             void* d_workspace, size_t workspace_bytes, void* stream);

/*
 * Trace mode of one layer over a batch: per neuron and queue column, the register after
 * the step, the step's spike / overflow flags and the time of the event it processed
 * (run_layer_traced, salt_core/quant/scan.py:83-132; LayerForwardTrace and event_ms,
 * salt_core/trace.py:13-55).  steps = max_queue_len for conv, L for FC; outputs are
 * [B][n][steps]: d_v_steps int32, d_event_ms float32 (NaN for columns past the neuron's
 * real events: catch-up and identity columns), d_flags uint8 (bit 0 spike, bit 1
 * register overflow before write-back).  A debug path (one thread per neuron).
 */
int32_t salt_layer_trace(const salt_layer_desc* desc, const salt_qparams* prm,
                         const salt_events_in* in, int32_t steps, int32_t* d_v_steps,
                         float* d_event_ms, uint8_t* d_flags, void* stream);

/*
 * salt_layer_forward without a workspace argument and without any device allocation.
 * It has no counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 * The workspace is a static per-device scratch array of SALT_STATIC_SCRATCH_BYTES, held
 * from the library's load until the process ends; a layer and batch that need more
 * (salt_layer_workspace_size) are rejected with -1 and a message.  Every call on one
 * device shares that device's array, which keeps the last call's contents (the call
 * clears what must start at zero): calls that overlap on one device race, so issue them
 * on one stream, or synchronise between streams.  Inputs, outputs and results are the
 * caller's, as for salt_layer_forward.
 */
#define SALT_STATIC_SCRATCH_BYTES ((size_t)64 << 20)
int32_t salt_layer_forward_static(const salt_layer_desc* desc, const salt_qparams* prm,
                                  const salt_events_in* in, const salt_events_out* out,
                                  const salt_layer_result* result, void* stream);

/* Order-sensitive 64-bit hash per stream, for streams too large to copy back.
 * With mix64 = the splitmix64 finaliser (add 0x9E3779B97F4A7C15, then xor-shift-multiply
 * by 0xBF58476D1CE4E5B9 and 0x94D049BB133111EB), entry i < min(n, cap) contributes
 * mix64(mix64(i) ^ (bits(time_i) << 32 | src_i)); the contributions are summed mod 2^64
 * and hash = mix64(sum + n * 0x2545F4914F6CDD1D).  d_hash: [B] uint64. */
int32_t salt_stream_hash(const float* d_times, const int32_t* d_src, const int32_t* d_n,
                         int32_t B, int32_t cap, uint64_t* d_hash, void* stream);

#ifdef __cplusplus
}
#endif
#endif
