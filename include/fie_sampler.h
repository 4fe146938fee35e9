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
 * Conventions: every pointer in the argument struct is a DEVICE pointer; work is
 * enqueued on `stream` (a hipStream_t passed as void*, NULL = the null stream) and
 * nothing synchronises; functions return FIE_OK or a negative FIE_E* code and never
 * throw.  The workspace is caller-owned device memory that needs no clearing: every
 * call writes what it later reads.  Calls that share a workspace must be ordered on
 * one stream.  The library allocates no device memory.
 *
 * Limits: 1 <= vocab <= 524288 (at most 64 tiles of 8192 tokens per row), rows >= 0,
 * token ids in penalty histories >= 0.
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

/* Per-row flags (fie_sampler_args.flags). */
enum {
    FIE_FLAG_GREEDY = 1,    /* SamplingParams.greedy (sampling.py:71-74) */
    FIE_FLAG_PENALTY = 2,   /* SamplingParams.has_penalties (sampling.py:76-79) */
};

/* Per-row status bits written to fie_sampler_args.status (informational). */
enum {
    FIE_ROW_OK = 0,
    FIE_ROW_EXACT_PATH = 1,      /* resolved by the full-row re-read path: the
                                    answer lay outside the streamed candidates */
    FIE_ROW_UNCOUNTED_IDS = 2,   /* the history held ids >= vocab but hist_invalid
                                    was NULL, so token 0's penalty (Q1) may differ */
};

typedef struct fie_sampler_args {
    /* logits [rows, vocab] in the engine dtype, rows `row_stride` elements apart.
       Borrowed and never written (sampler.py:108 works on a copy). */
    const void* logits;
    int32_t dtype;              /* FIE_F32 / FIE_F16 / FIE_BF16 */
    int32_t rows;
    int32_t vocab;
    int32_t lp_cols;            /* columns of top_ids/top_logprobs, 0..20 */
    int64_t row_stride;

    /* Per-row parameters, resolved the way sampler.py:182-192 resolves them. */
    const float* scale;         /* divisor: fp32(temperature), 1.0 for greedy rows */
    const int32_t* top_k;       /* 0 = off (also off for greedy rows and k >= vocab) */
    const float* top_p;         /* fp32(top_p); 1.0 = off */
    const float* min_p;         /* fp32(min_p); 0 = off */
    const int32_t* flags;       /* FIE_FLAG_* bits */
    const int32_t* logprobs;    /* -1 = no logprobs, else the row's count 0..20; may be
                                   NULL when no row asks for logprobs */
    const double* uniform;      /* caller-supplied draw in [0,1) per row; may be NULL
                                   when `rng` is given */

    /* Penalties (sampler.py:109-110,120-175).  apply_penalties is the batch gate
       "some row has penalties and contexts were passed"; the history is CSR and
       only rows with FIE_FLAG_PENALTY are read. */
    int32_t apply_penalties;
    int32_t max_row_hist;          /* largest history length of one row (host value);
                                      above 65535 the kernels count in 32 bits */
    const float* repetition;
    const float* presence;
    const float* frequency;
    const int64_t* hist_offsets;   /* [rows+1]: row r's ids are hist_ids[offsets[r], offsets[r+1]),
                                      or [offsets[r], hist_ends[r]) when hist_ends is given */
    const int32_t* hist_ids;       /* each id >= 0 */
    /* [rows] or NULL.  For a row whose history holds ids >= vocab: the number of
       distinct such ids, plus (1 << 30) if one of them first occurs after the first
       occurrence of token 0.  NULL means no id >= vocab occurs (checked: a row that
       breaks this gets FIE_ROW_UNCOUNTED_IDS). */
    const int32_t* hist_invalid;

    /* Outputs.  Only tokens is required; every other pointer may be NULL. */
    int64_t* tokens;            /* [rows] chosen token ids */
    int32_t* status;            /* [rows] FIE_ROW_* bits */
    uint32_t* tk_key;           /* [rows] order key of the top-k threshold value (0 = none) */
    uint64_t* cut_comp;         /* [rows] (key<<32 | ~index) of the last top-p survivor (0 = none) */
    float* row_max;             /* [rows] largest scaled logit M */
    uint64_t* kept_mass;        /* [rows*2] kept mass, low and high 64 bits */
    uint64_t* row_mass;         /* [rows*2] mass of the whole row (rows that need it) */
    float* chosen_logprob;      /* [rows] (rows with logprobs >= 0) */
    int64_t* top_ids;           /* [rows, lp_cols] (-1 past the row's count) */
    float* top_logprobs;        /* [rows, lp_cols] */

    /* On-device draws (optional; replaces the per-request generators of
       sampler.py:58-73).  When non-NULL, row r's uniform is derived on the device
       from rng[3r .. 3r+2] = (key0, key1, counter): the first 64-bit word x of the
       Philox4x64-10 block (Salmon et al., SC 2011) at counter (counter, 0, 0, 0) and
       key (key0, key1), as (x >> 11) * 2^-53, and `uniform` is not read.  The
       caller keeps one key per stream and advances its counter per draw. */
    const uint64_t* rng;

    /* [rows] or NULL: explicit ends of the rows' histories, for a history that
       lives in one device array across steps (rows in any order, non-contiguous);
       hist_offsets then holds the starts [rows]. */
    const int64_t* hist_ends;
} fie_sampler_args;

/* Device workspace owned by the caller: `bytes` of device memory at `ptr`
   (256-byte aligned), valid for calls with at most `max_rows` rows and a
   vocabulary of at most `vocab`. */
typedef struct fie_workspace {
    void* ptr;
    size_t bytes;
    int32_t max_rows;
    int32_t vocab;
} fie_workspace;

/* Bytes of workspace for calls with at most `max_rows` rows and a vocabulary of at
   most `vocab` (0 on invalid sizes).  A workspace for at most 16 rows also holds the
   arrays of the per-row kernel's span helpers (about 1.7 MiB a row at vocab 151936):
   calls of at most 16 rows in such a workspace settle rows the candidates cannot
   settle with one extra workgroup per 8192-token span of each sampled row. */
size_t fie_sampler_workspace_size(int32_t max_rows, int32_t vocab);

/* One sampler step: sampler.py:81-117 minus host bookkeeping.  Up to four kernels:
   the penalty histories bucketed by span, one streaming read of the logits, one
   workgroup per row, then the rows the candidates could not settle (with no more
   rows than the GPU has CUs, the per-row kernel settles those itself and the fourth
   is not launched). */
int fie_sampler_sample(const fie_sampler_args* args, const fie_workspace* ws, void* stream);

/* fie_sampler_sample with the model's output projection fused in front of it.  The
   reference computes the logits as `self._lm_head()(hidden)`, an nn.Linear without bias
   in the model dtype (continuous_batching.py:1345,1594,2225), and passes that buffer to
   the sampler (:1926-1928).  Here one kernel computes args->logits = hidden · weightᵀ
   (fp32 accumulation, rounded to nearest even in args->dtype, which must be FIE_F16 or
   FIE_BF16, the dtype of hidden and weight) and, from the values it wrote, the
   per-tile partials the sampler's streaming pass would read back; the rest of the
   chain is fie_sampler_sample's.  args->logits is written (row stride args->row_stride)
   and must hold rows x vocab.  hidden: [rows, hidden_dim] row-major; weight:
   [vocab, hidden_dim] row-major (nn.Linear's layout); both 16-byte aligned, and
   hidden_dim a multiple of 128. */
int fie_sampler_lmhead_sample(const fie_sampler_args* args, const void* hidden, const void* weight,
                              int32_t hidden_dim, const fie_workspace* ws, void* stream);

/* The fused kernel of fie_sampler_lmhead_sample alone (no penalty bucketing before it,
   no selection after it), with the same arguments.  No counterpart in the reference:
   it exists so a profiler or a benchmark can time the fused kernel by itself, after
   one whole fie_sampler_lmhead_sample has prepared the workspace. */
int fie_sampler_lmhead_stage(const fie_sampler_args* args, const void* hidden, const void* weight,
                             int32_t hidden_dim, const fie_workspace* ws, void* stream);

/* The kernels of fie_sampler_sample, one at a time, in this order (same args and
   workspace each time).  No counterpart in the reference: it exists so a profiler
   or a benchmark can time each kernel of the chain separately. */
enum {
    FIE_STAGE_PREP = 0,        /* the penalty histories bucketed by span (no-op without penalties) */
    FIE_STAGE_SCAN = 1,        /* the streaming pass over the logits */
    FIE_STAGE_FINISH = 2,      /* the per-row selection and draw from the candidates */
    FIE_STAGE_DEEP = 3,        /* the rows FINISH queued: passes over the whole row (no-op when none;
                                  FINISH queues none when rows <= the GPU's CUs) */
};
int fie_sampler_stage(const fie_sampler_args* args, const fie_workspace* ws, int32_t stage,
                      void* stream);

/* Greedy fast path, sampler.py:103-106: logits.argmax(-1), first index on ties. */
int fie_sampler_argmax(const void* logits, int32_t dtype, int32_t rows, int32_t vocab,
                       int64_t row_stride, int64_t* tokens, const fie_workspace* ws,
                       void* stream);

/* Kept set and normalised probabilities of the last fie_sampler_sample on this
   workspace (same args): kept[r*vocab+i] = 1 if token i survived _filter
   (sampler.py:187-229), probs = the draw distribution over the kept set.  A
   verification aid with no counterpart in the reference; either output may be
   NULL. */
int fie_sampler_kept(const fie_sampler_args* args, uint8_t* kept, float* probs,
                     const fie_workspace* ws, void* stream);

/* The build's canonical fp32 exponential on n device values (verification aid). */
int fie_sampler_cexp(const float* in, float* out, int64_t n, void* stream);

/* ids[dst[i]] = src[i] for i < n: appends new tokens to penalty histories kept in
   one device array across steps (no counterpart in the reference, whose history is
   repacked on the host every step, sampler.py:134-155). */
int fie_sampler_history_write(int32_t* ids, const int64_t* dst, const int32_t* src, int64_t n,
                              void* stream);

/* The on-device uniforms of `rng` (see fie_sampler_args) for `rows` rows into
   out[rows] (verification; no counterpart in the reference). */
int fie_sampler_uniforms(const uint64_t* rng, double* out, int32_t rows, void* stream);

/* Message of the last failing call on this thread (static storage). */
const char* fie_sampler_last_error(void);

/* fie_sampler_sample without a caller workspace and without any allocation: the
 * kernels use a static device array of FIE_SCRATCH_BYTES (64 MiB), resolved once
 * per device on the first call there and held by each device until the process
 * ends.  No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops).  Returns
 * FIE_E_WORKSPACE when fie_sampler_workspace_size(rows, vocab) exceeds the array
 * (for at most 16 rows: when it does even without the span helpers' arrays, which
 * are then left out and the rows settled without helpers).
 * Calls that overlap on one device share the array and race; calls on one stream,
 * or otherwise ordered, are safe. */
#define FIE_SCRATCH_BYTES ((size_t)64 << 20)
int fie_sampler_sample_noalloc(const fie_sampler_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FIE_SAMPLER_H */
