/*
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product may load or call this file;
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and
 * only as the checker.
 *
 * Plain-C restatement of the reference token sampler
 *   engine/batching/sampler.py:81-291  (BatchedSampler.sample and its stages)
 *   engine/runtime/sampling.py:71-79   (greedy / has_penalties predicates)
 * written as the checker for the HIP sampler.  Each stage follows the reference
 * line it cites.  Where the reference leaves a result to ATen's float rounding
 * (the fp32 bits of softmax and cumsum that decide a top-p boundary, the tie order
 * of an unstable sort, the torch.multinomial stream), the build's canonical rules
 * replace it:
 *
 *   (R1) weights   The row is cut into tiles: token 0 alone, then
 *                  [1, T), [T, 2T), ... with T = FIE_TILE.  m_t is the largest
 *                  scaled logit of tile t and M the largest of the row.
 *                    W_i = floor(cexp(y_i - m_t) * 2^40)      (token weight)
 *                    C_t = floor(cexp(m_t - M)  * 2^40)      (tile scale)
 *                    w_i = W_i * C_t                          (row weight, < 2^81)
 *                  Every mass is an exact integer sum of w_i, so no summation
 *                  order matters, and a tile's sums need only its own maximum.
 *   (R2) order     tokens rank by (y descending, token index ascending).
 *   (R3) top-p     the token at rank j is dropped iff  sum_{rank<j} w >= ceil(p*S)
 *                  (S = mass of the top-k/min-p survivors, p the fp32 top_p),
 *                  evaluated exactly.
 *   (R4) draw      t = floor(u * K) with K the kept mass; the token is the first
 *                  kept token in (R2) order whose inclusive prefix mass exceeds t.
 *   (R5) min-p     a token is dropped iff fl(y_i - M) < L, where L is the fp32
 *                  found by a 32-step bisection over order keys on [-80, 0] for
 *                  the boundary of cexp(d) >= fp32(min_p) (oracle_minp_bound).
 *                  Exactly the reference's probs < max(probs) * min_p in real
 *                  arithmetic; the bisection makes the kept set a prefix of the
 *                  value order even where cexp's last bit is not monotone.
 *   (R6) top_p==1  drops nothing (the exact-arithmetic reading of the reference's
 *                  `cumulative - p >= 1.0` test, sampler.py:226).
 *   (R7) logprobs  lse = M + ln(S_all) - 80 ln 2, S_all the mass of the whole row.
 *
 * cexp() is the build's own fp32 exponential: Cody-Waite reduction by ln 2 (split
 * constant), a degree-7 Taylor polynomial for e^r on |r| <= ln2/2 evaluated by
 * Horner with fused multiply-adds, and an exact scaling by 2^n.  Every operation is
 * an IEEE-754 binary32 operation with round-to-nearest-even, so the HIP kernels,
 * which perform the same operations in the same order, produce the same bits.
 * Compile with -ffp-contract=off so the compiler adds no fusions of its own.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define FIE_TILE 2048
typedef unsigned __int128 u128;

/* ------------------------------------------------------------------ arithmetic */

float oracle_cexp(float d)
{
    if (!(d > -80.0f)) return 0.0f;          /* -inf, NaN and deep underflow */
    if (d >= 0.0f) return 1.0f;              /* y - M is never positive */
    float n = rintf(d * 1.44269502f);        /* round(d / ln 2) */
    float r = fmaf(n, -0.693145752f, d);     /* ln2 high part, 16 significant bits */
    r = fmaf(n, -1.42860677e-06f, r);        /* ln2 low part */
    float p = 1.98412701e-04f;               /* 1/7! */
    p = fmaf(p, r, 1.38888892e-03f);         /* 1/6! */
    p = fmaf(p, r, 8.33333377e-03f);         /* 1/5! */
    p = fmaf(p, r, 4.16666679e-02f);         /* 1/4! */
    p = fmaf(p, r, 1.66666672e-01f);         /* 1/3! */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

/* cexp() over every fp32 d in [lo, hi] (bit patterns walked in order): returns the
 * number of adjacent pairs where the result decreases as d increases. */
int64_t oracle_cexp_monotone_violations(float lo, float hi)
{
    int64_t bad = 0;
    float prev = oracle_cexp(lo);
    float d = lo;
    while (d < hi) {
        d = nextafterf(d, hi);
        float e = oracle_cexp(d);
        if (e < prev) ++bad;
        prev = e;
    }
    return bad;
}

static inline float key_float(uint32_t k)
{
    uint32_t b = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

static inline uint32_t fkey_(float y)
{
    uint32_t b;
    memcpy(&b, &y, 4);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

/* Rule R5's bound: bisection over the order keys of d in [-80, 0] with the
 * predicate cexp(d) >= mp (false at -80 unless mp is tiny, true at 0); returns the
 * smallest d the bisection lands on, or -inf when every d passes. */
float oracle_minp_bound(float mp)
{
    uint32_t lo = fkey_(-80.0f), hi = fkey_(0.0f);
    if (oracle_cexp(key_float(lo)) >= mp) return -INFINITY;
    while (hi - lo > 1) {
        uint32_t mid = lo + (hi - lo) / 2;
        if (oracle_cexp(key_float(mid)) >= mp) hi = mid;
        else lo = mid;
    }
    return key_float(hi);
}

static inline uint64_t fixed40(float e)
{
    return (uint64_t)((double)e * 1099511627776.0);   /* floor(e * 2^40), exact */
}

/* Order-preserving key of an fp32 value: larger value, larger key. */
static inline uint32_t fkey(float y)
{
    uint32_t b;
    memcpy(&b, &y, 4);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

/* (R2): descending composite = descending value, then ascending index. */
static inline uint64_t comp_of(float y, int32_t idx)
{
    return ((uint64_t)fkey(y) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)idx);
}

static inline int32_t idx_of(uint64_t comp)
{
    return (int32_t)(0xFFFFFFFFu - (uint32_t)(comp & 0xFFFFFFFFu));
}

static int cmp_desc_u64(const void* a, const void* b)
{
    uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
    return (x < y) - (x > y);
}

/* floor(m * X / 2^q) for m < 2^53, X < 2^128, exactly (a 192-bit product). */
static u128 mul_shift(uint64_t m, u128 X, int q)
{
    u128 lo = (u128)m * (uint64_t)X;                     /* < 2^117 */
    u128 hi = (u128)m * (uint64_t)(X >> 64);             /* < 2^117 */
    /* product = hi * 2^64 + lo = P2 * 2^128 + P1 * 2^64 + P0 */
    uint64_t p0 = (uint64_t)lo;
    u128 mid = (lo >> 64) + hi;                          /* < 2^118 */
    uint64_t p1 = (uint64_t)mid;
    uint64_t p2 = (uint64_t)(mid >> 64);
    if (q >= 192) return 0;
    if (q >= 128) return (u128)(p2 >> (q - 128));
    if (q >= 64) {
        int s = q - 64;
        u128 v = ((u128)p2 << 64) | p1;
        return s ? (v >> s) : v;
    }
    u128 v = ((u128)p1 << 64) | p0;
    return q ? ((v >> q) | ((u128)p2 << (128 - q))) : v;
}

/* Exact ceil(p * S) for an fp32 p in (0, 1) and S < 2^128 (a 192-bit product). */
static u128 ceil_mul_f32(float p, u128 S)
{
    uint32_t b;
    memcpy(&b, &p, 4);
    uint32_t eb = (b >> 23) & 0xFFu;
    uint64_t mant = (b & 0x7FFFFFu) | (eb ? 0x800000u : 0u);
    int q = eb ? 150 - (int)eb : 149;                    /* p = mant / 2^q, q >= 24 */
    u128 fl = mul_shift(mant, S, q);                     /* floor(mant S / 2^q) */
    u128 low = mul_shift(mant, S, 0);                    /* mant S mod 2^128 */
    int frac;
    if (q < 128) {
        frac = (low & ((((u128)1) << q) - 1)) != 0;
    } else {
        u128 mid = mul_shift(mant, S, 128);              /* mant S >> 128 */
        frac = low != 0 || (mid & ((((u128)1) << (q - 128)) - 1)) != 0;
    }
    return fl + (frac ? 1 : 0);
}

/* Exact floor(u * K) for a double u in [0, 1) and K < 2^104. */
static u128 floor_mul_f64(double u, u128 K)
{
    if (!(u > 0.0)) return 0;
    uint64_t b;
    memcpy(&b, &u, 8);
    uint32_t eb = (uint32_t)((b >> 52) & 0x7FFu);
    uint64_t mant = (b & 0xFFFFFFFFFFFFFull) | (eb ? (1ull << 52) : 0ull);
    int q = eb ? 1075 - (int)eb : 1074;                  /* u = mant / 2^q */
    return mul_shift(mant, K, q);
}

/* u128 -> double as hi * 2^64 + lo, both conversions and the add in double. */
static double u128_to_double(u128 x)
{
    return (double)(uint64_t)(x >> 64) * 18446744073709551616.0 + (double)(uint64_t)x;
}

/* ------------------------------------------------------------------ penalties */

typedef struct { int32_t id; int32_t pos; } occ_t;
typedef struct { int32_t id; int32_t count; int32_t first; } uniq_t;

static int cmp_occ(const void* a, const void* b)
{
    const occ_t *x = a, *y = b;
    if (x->id != y->id) return (x->id > y->id) - (x->id < y->id);
    return (x->pos > y->pos) - (x->pos < y->pos);
}

static int cmp_first(const void* a, const void* b)
{
    const uniq_t *x = a, *y = b;
    return (x->first > y->first) - (x->first < y->first);
}

/* Distinct ids of one context in first-occurrence order with their counts, exactly
 * the insertion order of the reference's `occurrences` dict (sampler.py:140-144). */
static int32_t unique_in_order(const int32_t* ids, int64_t n, uniq_t* out, occ_t* tmp)
{
    for (int64_t i = 0; i < n; ++i) { tmp[i].id = ids[i]; tmp[i].pos = (int32_t)i; }
    qsort(tmp, (size_t)n, sizeof(occ_t), cmp_occ);
    int32_t u = 0;
    for (int64_t i = 0; i < n; ++i) {
        if (i == 0 || tmp[i].id != tmp[i - 1].id) {
            out[u].id = tmp[i].id; out[u].count = 1; out[u].first = tmp[i].pos; ++u;
        } else {
            out[u - 1].count += 1;
        }
    }
    qsort(out, (size_t)u, sizeof(uniq_t), cmp_first);
    return u;
}

/*
 * _apply_penalties, sampler.py:120-175, in place on w[B*V].
 * The gather reads the unpenalised logits; the scatter then writes, for every row,
 * `width` entries in column order (real entries first, pad entries after), and a
 * later write to the same index replaces an earlier one, as a sequential CPU
 * scatter does.  Pad entries and ids >= V target index 0 with the original logit of
 * token 0 (sampler.py:156-157,174), which is how a real token-0 penalty can be
 * undone (Q1).  Rows without penalties or with an empty context contribute no
 * entries (sampler.py:136-139).  Returns the batch width, or -1 on a negative id.
 */
int32_t oracle_penalize(float* w, int32_t B, int32_t V, const uint8_t* has_pen,
                        const float* rep, const float* pres, const float* freq,
                        const int64_t* off, const int32_t* ids)
{
    int64_t maxn = 0;
    for (int32_t r = 0; r < B; ++r) {
        int64_t n = off[r + 1] - off[r];
        if (n > maxn) maxn = n;
        for (int64_t i = off[r]; i < off[r + 1]; ++i) if (ids[i] < 0) return -1;
    }
    if (B <= 0) return 0;
    uniq_t** rows = calloc((size_t)(uint32_t)B, sizeof(uniq_t*));
    int32_t* nu = calloc((size_t)(uint32_t)B, sizeof(int32_t));
    occ_t* tmp = malloc((size_t)(maxn ? maxn : 1) * sizeof(occ_t));
    int32_t width = 0;
    for (int32_t r = 0; r < B; ++r) {
        int64_t n = off[r + 1] - off[r];
        if (!has_pen[r] || n == 0) continue;
        rows[r] = malloc((size_t)n * sizeof(uniq_t));
        nu[r] = unique_in_order(ids + off[r], n, rows[r], tmp);
        if (nu[r] > width) width = nu[r];
    }
    if (width > 0) {
        float* src = malloc((size_t)width * sizeof(float));
        int32_t* dst = malloc((size_t)width * sizeof(int32_t));
        for (int32_t r = 0; r < B; ++r) {
            float* row = w + (int64_t)r * V;
            float g0 = row[0];
            /* gather every value first: the scatter source is built from the input */
            for (int32_t j = 0; j < width; ++j) {
                if (j < nu[r] && rows[r][j].id < V) {
                    float g = row[rows[r][j].id];
                    float pen = (g > 0.0f) ? g / rep[r] : g * rep[r];
                    pen = pen - pres[r];
                    pen = pen - freq[r] * (float)rows[r][j].count;
                    src[j] = pen;
                    dst[j] = rows[r][j].id;
                } else {
                    src[j] = g0;
                    dst[j] = 0;
                }
            }
            for (int32_t j = 0; j < width; ++j) row[dst[j]] = src[j];
        }
        free(src); free(dst);
    }
    for (int32_t r = 0; r < B; ++r) free(rows[r]);
    free(rows); free(nu); free(tmp);
    return width;
}

/* ------------------------------------------------------------------ one step */

typedef struct {
    int32_t B, V;
    float* logits;                 /* [B*V] fp32, modified in place by penalties */
    const float* scale;            /* divisor: fp32(temperature), 1.0 for greedy rows */
    const int32_t* top_k;          /* effective k, 0 = off */
    const float* top_p;            /* effective p, 1.0 = off */
    const float* min_p;            /* effective min_p, 0 = off */
    const uint8_t* greedy;
    const int32_t* logprobs;       /* -1 = none, else 0..20 */
    const double* uniform;         /* [B], in [0,1) */
    int32_t apply_penalties;
    const uint8_t* has_pen;
    const float *rep, *pres, *freq;
    const int64_t* hist_off;       /* [B+1] */
    const int32_t* hist_ids;
    int32_t lp_cols;               /* columns of top_ids/top_lp */
    /* outputs */
    int64_t* tokens;               /* [B] */
    uint32_t* tk_key;              /* [B] key of the top-k threshold value (0 = none) */
    uint64_t* cut_comp;            /* [B] composite of the last top-p survivor (0 = none) */
    float* row_max;                /* [B] M */
    uint64_t* kept_mass;           /* [B*2] kept mass, low and high 64 bits */
    uint64_t* row_mass;            /* [B*2] whole-row mass, low and high 64 bits */
    uint8_t* kept;                 /* [B*V] or NULL */
    float* probs;                  /* [B*V] or NULL */
    float* chosen_lp;              /* [B] or NULL */
    int64_t* top_ids;              /* [B*lp_cols] or NULL */
    float* top_lp;                 /* [B*lp_cols] or NULL */
} oracle_args;

static inline int tile_of(int32_t i) { return i == 0 ? 0 : 1 + i / FIE_TILE; }

int32_t oracle_sample(oracle_args* a)
{
    const int32_t B = a->B, V = a->V;
    if (V <= 0 || V >= (1 << 24)) return -2;
    if (a->apply_penalties) {
        if (oracle_penalize(a->logits, B, V, a->has_pen, a->rep, a->pres, a->freq,
                            a->hist_off, a->hist_ids) < 0) return -1;
    }
    const int NTS = 2 + (V - 1) / FIE_TILE;             /* tile slots incl. token 0 */
    float* y = malloc((size_t)V * sizeof(float));
    u128* w = malloc((size_t)V * sizeof(u128));
    uint64_t* order = malloc((size_t)V * sizeof(uint64_t));
    uint8_t* surv = malloc((size_t)V);
    uint32_t* tmax = malloc((size_t)NTS * sizeof(uint32_t));
    uint64_t* tC = malloc((size_t)NTS * sizeof(uint64_t));
    for (int32_t r = 0; r < B; ++r) {
        const float* xr = a->logits + (int64_t)r * V;
        const float s = a->scale[r];
        /* _apply_temperature, sampler.py:177-185: a true fp32 divide per element */
        for (int t = 0; t < NTS; ++t) tmax[t] = 0;      /* 0 = empty tile */
        uint32_t best = 0;
        int32_t amax = 0;
        for (int32_t i = 0; i < V; ++i) {
            y[i] = xr[i] / s + 0.0f;                     /* +0.0f folds -0 into +0 */
            uint32_t k = fkey(y[i]);
            if (i == 0 || k > best) { best = k; amax = i; }
            int t = tile_of(i);
            if (k > tmax[t]) tmax[t] = k;      /* keys of non-NaN values are never 0 */
        }
        const float M = y[amax];
        a->row_max[r] = M;
        /* (R1) tile scales and row weights */
        for (int t = 0; t < NTS; ++t) {
            if (tmax[t] == 0) { tC[t] = 0; continue; }
            uint32_t kt = tmax[t];
            uint32_t bits = (kt & 0x80000000u) ? (kt & 0x7FFFFFFFu) : ~kt;
            float mt;
            memcpy(&mt, &bits, 4);
            tC[t] = fixed40(oracle_cexp(mt - M));
        }
        u128 sall = 0;
        for (int32_t i = 0; i < V; ++i) {
            const int t = tile_of(i);
            uint32_t kt = tmax[t];
            uint32_t bits = (kt & 0x80000000u) ? (kt & 0x7FFFFFFFu) : ~kt;
            float mt;
            memcpy(&mt, &bits, 4);
            w[i] = (u128)fixed40(oracle_cexp(y[i] - mt)) * tC[t];
            sall += w[i];
        }
        a->row_mass[2 * r] = (uint64_t)sall;
        a->row_mass[2 * r + 1] = (uint64_t)(sall >> 64);
        a->tk_key[r] = 0;
        a->cut_comp[r] = 0;
        int need_sort = a->greedy[r] ? (a->logprobs[r] > 0) : 1;
        if (need_sort) {
            for (int32_t i = 0; i < V; ++i) order[i] = comp_of(y[i], i);
            qsort(order, (size_t)V, sizeof(uint64_t), cmp_desc_u64);
        }
        u128 T = 0;
        if (a->greedy[r]) {
            /* _draw greedy rows, sampler.py:236-238: argmax, first index on ties */
            a->tokens[r] = amax;
            T = w[amax];
            if (a->kept) memset(a->kept + (int64_t)r * V, 1, (size_t)V);
            if (a->probs) {
                memset(a->probs + (int64_t)r * V, 0, (size_t)V * sizeof(float));
                a->probs[(int64_t)r * V + amax] = 1.0f;
            }
        } else {
            /* _filter top-k, sampler.py:194-209: keep y >= k-th largest value */
            uint32_t tk = 0;
            if (a->top_k[r] > 0) {
                tk = (uint32_t)(order[a->top_k[r] - 1] >> 32);
                a->tk_key[r] = tk;
            }
            /* _filter min-p, sampler.py:211-218, rule (R5) */
            const float mp = a->min_p[r];
            const float L = mp > 0.0f ? oracle_minp_bound(mp) : -INFINITY;
            u128 S = 0;
            for (int32_t i = 0; i < V; ++i) {
                surv[i] = (fkey(y[i]) >= tk) && !(mp > 0.0f && (y[i] - M) < L);
                if (surv[i]) S += w[i];
            }
            /* _filter top-p, sampler.py:220-228, rules (R2)(R3)(R6) */
            const float p = a->top_p[r];
            if (p < 1.0f) {
                u128 thr = ceil_mul_f32(p, S);
                u128 excl = 0;
                int stopped = 0;
                for (int32_t j = 0; j < V; ++j) {
                    int32_t i = idx_of(order[j]);
                    if (!surv[i]) continue;
                    if (stopped || excl >= thr) { stopped = 1; surv[i] = 0; continue; }
                    excl += w[i];
                    a->cut_comp[r] = order[j];
                }
            }
            for (int32_t i = 0; i < V; ++i) if (surv[i]) T += w[i];
            /* _draw sampled rows, sampler.py:241-259, replaced by rule (R4) */
            int64_t tok = amax;
            if (T > 0) {
                u128 t = floor_mul_f64(a->uniform[r], T);
                u128 incl = 0;
                for (int32_t j = 0; j < V; ++j) {
                    int32_t i = idx_of(order[j]);
                    if (!surv[i]) continue;
                    incl += w[i];
                    if (incl > t) { tok = i; break; }
                }
            }
            a->tokens[r] = tok;
            if (a->kept) for (int32_t i = 0; i < V; ++i) a->kept[(int64_t)r * V + i] = surv[i];
            if (a->probs) {
                double Td = u128_to_double(T);
                for (int32_t i = 0; i < V; ++i)
                    a->probs[(int64_t)r * V + i] =
                        (surv[i] && T > 0) ? (float)(u128_to_double(w[i]) / Td) : 0.0f;
            }
        }
        a->kept_mass[2 * r] = (uint64_t)T;
        a->kept_mass[2 * r + 1] = (uint64_t)(T >> 64);
        /* _logprobs, sampler.py:262-291, rule (R7) */
        if (a->logprobs[r] >= 0) {
            double lse = log(u128_to_double(sall)) - 80.0 * 0.69314718055994530942;
            if (a->chosen_lp) {
                int64_t c = a->tokens[r];
                a->chosen_lp[r] = (float)(((double)y[c] - (double)M) - lse);
            }
            if (a->top_ids) {
                for (int32_t j = 0; j < a->lp_cols; ++j) {
                    int64_t o = (int64_t)r * a->lp_cols + j;
                    if (j < a->logprobs[r] && j < V) {
                        int32_t i = idx_of(order[j]);
                        a->top_ids[o] = i;
                        a->top_lp[o] = (float)(((double)y[i] - (double)M) - lse);
                    } else {
                        a->top_ids[o] = -1;
                        a->top_lp[o] = 0.0f;
                    }
                }
            }
        }
    }
    free(y); free(w); free(order); free(surv); free(tmax); free(tC);
    return 0;
}

/* ------------------------------------------------------------------ division check */

static float f16_to_f32(uint16_t h)
{
    uint32_t sgn = (h >> 15) & 1u, e = (h >> 10) & 31u, m = h & 1023u;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(m | 1024u), (int)e - 25);
    return sgn ? -v : v;
}

static float markstein(float x, float s, float r)
{
    float q = x * r;
    float e = fmaf(-q, s, x);
    return fmaf(e, r, q);
}

/* The HIP kernels divide by the temperature with Markstein's correction
 * q = RN(x r), e = x - q s, RN(q + e r) from r = RN(1/s) when 2^-96 <= |x| <= 2^96
 * and 2^-30 <= s <= 2^30.  Counts, for one s, the inputs in that range where it
 * differs from the IEEE quotient: every fp16 value, every bf16 value, and
 * `nrandom` pseudo-random fp32 values (xorshift from `seed`). */
int64_t oracle_markstein_mismatches(float s, int64_t nrandom, uint32_t seed)
{
    const float r = 1.0f / s;
    int64_t bad = 0;
    for (uint32_t h = 0; h < 65536u; ++h) {
        float xs[2];
        uint32_t bb = h << 16;
        xs[0] = f16_to_f32((uint16_t)h);
        memcpy(&xs[1], &bb, 4);
        for (int k = 0; k < 2; ++k) {
            float x = xs[k], a = fabsf(x);
            if (!(a >= 0x1p-96f && a <= 0x1p96f)) continue;
            float q1 = x / s, q2 = markstein(x, s, r);
            if (memcmp(&q1, &q2, 4) != 0) ++bad;
        }
    }
    uint32_t st = seed ? seed : 1u;
    for (int64_t i = 0; i < nrandom; ++i) {
        st ^= st << 13; st ^= st >> 17; st ^= st << 5;
        uint32_t e = 31u + (st % 193u);                  /* exponents 2^-96 .. 2^96 */
        uint32_t bits = (st & 0x807FFFFFu) | (e << 23);
        float x;
        memcpy(&x, &bits, 4);
        float q1 = x / s, q2 = markstein(x, s, r);
        if (memcmp(&q1, &q2, 4) != 0) ++bad;
    }
    return bad;
}
