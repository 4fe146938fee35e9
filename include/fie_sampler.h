/*
 * fie_sampler.h -- C ABI of the MI355X fused token sampler.
 *
 * The boundary replaces the device work of the reference's per-step sampler,
 * BatchedSampler.sample() (engine/batching/sampler.py:81-117), and its stages:
 *   penalties    _apply_penalties     sampler.py:120-175
 *   temperature  _apply_temperature   sampler.py:177-185
 *   filters      _filter              sampler.py:187-229  (top-k, min-p, top-p)
 *   draw         _draw                sampler.py:231-260  (argmax / inverse-CDF draw)
 *   logprobs     _logprobs            sampler.py:262-291
 * and the greedy fast path logits.argmax(-1) (sampler.py:103-106).
 *
 * Host-side validation, RNG ownership and the SampleResult type stay in the host
 * layer above this ABI (fie_amd/batching/sampler.py mirrors sampler.py:42-117).
 *
 * Conventions: every pointer in the argument structs is a DEVICE pointer unless its
 * comment says otherwise; work is enqueued on `stream` (a hipStream_t passed as
 * void*, NULL = the null stream) and nothing synchronises; functions return
 * FIE_OK or a negative FIE_E* code and never throw.  The workspace is caller-owned
 * device memory described by an fie_workspace, cleared once with
 * fie_sampler_workspace_init(); calls that share a workspace must be ordered on one
 * stream.  The library allocates no device memory.
 */
#ifndef FIE_SAMPLER_H
#define FIE_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    FIE_OK = 0,
    FIE_E_ARG = -1,        /* a size, pointer or dtype is invalid */
    FIE_E_WORKSPACE = -2,  /* workspace missing or too small */
    FIE_E_LAUNCH = -3,     /* a kernel launch failed (see fie_sampler_last_error) */
};

enum { FIE_F32 = 0, FIE_F16 = 1, FIE_BF16 = 2 };

/* Per-row status bits, OR-ed into fie_sampler_args.status (zero it before a call).
   Either bit means the row's outputs are not final: pass the row to
   fie_sampler_resolve_overflow.  After FIE_ROW_TIMEOUT also re-initialise the
   workspace before its next use. */
enum {
    FIE_ROW_OK = 0,
    FIE_ROW_OVERFLOW = 1,  /* candidate set exceeded the fast path's capacity */
    FIE_ROW_TIMEOUT = 2,   /* a bounded wait between the row's workgroups gave up */
};

typedef struct fie_sampler_args {
    /* logits [rows, vocab] in the engine dtype, rows `row_stride` elements apart.
       Borrowed and never written (sampler.py:108 works on a copy). */
    const void* logits;
    int32_t dtype;              /* FIE_F32 / FIE_F16 / FIE_BF16 */
    int32_t rows;
    int32_t vocab;
    int32_t lp_cols;            /* columns of top_ids/top_lp, 0..20 */
    int64_t row_stride;

    /* Per-row parameters, already resolved by the host layer the way
       sampler.py:182-192 resolves them. */
    const float* scale;         /* divisor: fp32(temperature), 1.0 for greedy rows */
    const int32_t* top_k;       /* 0 = off (also off for greedy rows and k >= vocab) */
    const float* top_p;         /* fp32(top_p); 1.0 = off */
    const float* min_p;         /* fp32(min_p); 0 = off */
    const int32_t* flags;       /* bit0 greedy, bit1 penalised row */
    const int32_t* logprobs;    /* -1 = no logprobs, else the row's count 0..20 */
    const double* uniform;      /* caller-supplied draw in [0,1) per row */

    /* Penalties (sampler.py:109-110,120-175).  apply_penalties is the batch gate
       "some row has penalties and contexts were passed"; history is CSR. */
    int32_t apply_penalties;
    int32_t reserved0;
    const float* repetition;
    const float* presence;
    const float* frequency;
    const int64_t* hist_offsets;   /* [rows+1] */
    const int32_t* hist_ids;       /* [hist_offsets[rows]], each id >= 0 */
    int64_t hist_total;            /* host copy of hist_offsets[rows] */
    int64_t epoch;                 /* strictly increasing per call on one workspace */

    /* Outputs. */
    int64_t* tokens;            /* [rows] chosen token ids */
    int32_t* status;            /* [rows] FIE_ROW_* bits, zeroed by the caller */
    uint32_t* tk_key;           /* [rows] order key of the top-k threshold value (0 = none) */
    uint64_t* cut_comp;         /* [rows] (key<<32 | ~index) of the last top-p survivor (0 = none) */
    float* row_max;             /* [rows] largest scaled logit M */
    uint64_t* kept_mass;        /* [rows] sum of kept weights floor(e^(y-M) * 2^40) */
    uint64_t* row_mass;         /* [rows] same sum over the whole row */
    float* chosen_logprob;      /* [rows] (rows with logprobs >= 0) */
    int64_t* top_ids;           /* [rows, lp_cols] (-1 past the row's count) */
    float* top_logprobs;        /* [rows, lp_cols] */
} fie_sampler_args;

/* Device workspace owned by the caller.  Its layout is fixed by (max_rows, vocab,
   max_hist); calls may use fewer rows, a smaller vocabulary and less history. */
typedef struct fie_workspace {
    void* ptr;                  /* device memory, 256-byte aligned */
    size_t bytes;               /* at least fie_sampler_workspace_size(...) */
    int32_t max_rows;
    int32_t vocab;              /* largest vocabulary used with this workspace */
    int64_t max_hist;           /* largest hist_total used with this workspace */
} fie_workspace;

/* Bytes of workspace for calls with at most `max_rows` rows, a vocabulary of at
   most `vocab` and at most `max_hist` history ids in total. */
size_t fie_sampler_workspace_size(int32_t max_rows, int32_t vocab, int64_t max_hist);

/* Clear a freshly allocated workspace, or one whose last call failed. */
int fie_sampler_workspace_init(const fie_workspace* ws, void* stream);

/* One sampler step: sampler.py:81-117 minus host bookkeeping. */
int fie_sampler_sample(const fie_sampler_args* args, const fie_workspace* ws, void* stream);

/* The kernels of fie_sampler_sample, one at a time, in this order (same args and
   workspace each time).  No counterpart in the reference: it exists so a profiler
   or a benchmark can time each kernel of the chain separately. */
enum {
    FIE_STAGE_PENALTY = 0,     /* history counts and penalised values; skipped when
                                  apply_penalties == 0 */
    FIE_STAGE_SAMPLE = 1,      /* the fused step: one read of the logits */
};
int fie_sampler_stage(const fie_sampler_args* args, const fie_workspace* ws, int32_t stage,
                      void* stream);

/* Exact fallback for rows whose status has FIE_ROW_OVERFLOW after
   fie_sampler_sample (same args and workspace, before any other call on it).
   `row_list` is a device array of `count` row indices. */
int fie_sampler_resolve_overflow(const fie_sampler_args* args, const int32_t* row_list,
                                 int32_t count, const fie_workspace* ws, void* stream);

/* Greedy fast path, sampler.py:103-106: logits.argmax(-1), first index on ties. */
int fie_sampler_argmax(const void* logits, int32_t dtype, int32_t rows, int32_t vocab,
                       int64_t row_stride, int64_t* tokens, const fie_workspace* ws,
                       void* stream);

/* Kept set and normalised probabilities of the last fie_sampler_sample on this
   workspace (same args): kept[r*vocab+i] = 1 if token i survived _filter
   (sampler.py:187-229), probs = the draw distribution over the kept set.  A
   verification aid; either output may be NULL. */
int fie_sampler_kept(const fie_sampler_args* args, uint8_t* kept, float* probs,
                     const fie_workspace* ws, void* stream);

/* The build's canonical fp32 exponential on n device values (verification aid). */
int fie_sampler_cexp(const float* in, float* out, int64_t n, void* stream);

/* Profiling aid, no counterpart in the reference: when `buffer` (device memory,
   rows * slices * 8 uint64) is not NULL, every later fie_sampler_sample records
   wall-clock timestamps at the phase boundaries of each (row, slice) workgroup.
   NULL switches it off. */
int fie_sampler_set_trace(void* buffer);

/* Message of the last failing call on this thread (static storage). */
const char* fie_sampler_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* FIE_SAMPLER_H */
