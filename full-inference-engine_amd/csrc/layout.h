// Workspace layout and kernel parameter block of the MI355X sampler.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace fie {

constexpr int kCountBins = 4096;   // pass-1 histogram: order key of w >> 20
constexpr int kCountShift = 20;
constexpr int kMassBins = 2048;    // pass-2 histogram: d = y - M on a linear grid
constexpr int kCap = 2048;         // candidates per buffer per row
constexpr int kMaxSlices = 256;    // workgroups per row
constexpr int kMinSlice = 4096;    // elements per slice, lower bound
constexpr int kMaxSlice = 32768;   // elements per slice, upper bound (LDS bitmap)
constexpr int kPatchLds = 1024;    // penalty patches staged in LDS per slice
constexpr int kPenThreads = 1024;
constexpr int kMaxPenWords = 8192; // penalty bitmap words: vocab <= 262144
constexpr int kFallbackRows = 4;   // rows resolved at once by the exact fallback

// Mode bits of the second and third passes.
enum : uint32_t {
    kM2CollectA = 1u,   // gather candidates with w-key >= keyA
    kM2Weights = 2u,    // integer weights of the whole row (row_mass)
    kM2MassHist = 4u,   // survivor mass histogram over d
    kM3CollectB = 1u,   // gather candidates inside the mass windows
};

enum : uint32_t { kKindGreedy = 0, kKindTopK = 1, kKindWide = 2 };

// Per-row state.  Accumulators are zero between calls: whoever consumes one
// (the last workgroup of a pass) restores it to zero.
struct RowState {
    unsigned long long maxpack;      // max of (wkey << 32 | ~index) over the row
    unsigned long long sall;         // sum of integer weights over the row
    unsigned long long thr;          // ceil(p * S), the top-p threshold
    unsigned long long S;            // survivor mass
    unsigned long long Awa;          // survivor mass in front of window 0
    unsigned long long Abc;          // survivor mass in front of the cut bin
    unsigned int minkey_inv;         // max of ~wkey (the row minimum)
    unsigned int arrive[3];          // workgroup arrivals per hand-off (+ kPlanReady)
    unsigned int nA, nB;             // candidates gathered
    float M, dscale;                 // row max of y; d-bin scale
    unsigned int keyA;               // rank candidates: w-key lower bound
    unsigned int wlo[2], whi[2];     // mass windows as w-key intervals
    int bc, nwin, wb0;               // cut bin, windows, last bin of window 0
    unsigned int overflow;
    unsigned int pad[3];
};
static_assert(sizeof(RowState) == 128, "RowState is 128 bytes");

struct PenMeta {
    int nvalid;        // distinct ids < vocab
    int nuniq;         // distinct ids, including ids >= vocab (sampler.py:143)
    int has0;          // token 0 is in the history
    int inval_after0;  // an id >= vocab first occurs after token 0's first occurrence
};

struct Layout {
    size_t rows, pen, wbatch, chist, mcnt, mmass, candA, candB, seg, pen_ids, pen_vals,
        pen_cnt, fb_keys, total;
};

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

inline Layout make_layout(int64_t max_rows, int64_t max_hist, int64_t vocab)
{
    Layout L{};
    size_t o = 0;
    auto take = [&](size_t bytes) {
        size_t at = o;
        o = align_up(o + bytes, 256);
        return at;
    };
    const size_t R = (size_t)(max_rows > 0 ? max_rows : 1);
    const size_t H = (size_t)(max_hist > 0 ? max_hist : 1);
    L.rows = take(R * sizeof(RowState));
    L.pen = take(R * sizeof(PenMeta));
    L.wbatch = take(sizeof(uint64_t));
    L.chist = take(R * kCountBins * sizeof(uint32_t));
    L.mcnt = take(R * kMassBins * sizeof(uint32_t));
    L.mmass = take(R * kMassBins * sizeof(uint64_t));
    L.candA = take(R * kCap * sizeof(uint64_t));
    L.candB = take(R * kCap * sizeof(uint64_t));
    L.seg = take(R * (kMaxSlices + 1) * sizeof(int32_t));
    L.pen_ids = take(H * sizeof(int32_t));
    L.pen_vals = take(H * sizeof(float));
    L.pen_cnt = take(H * sizeof(uint32_t));
    size_t vp = 64;
    while ((int64_t)vp < vocab) vp <<= 1;
    L.fb_keys = take((size_t)kFallbackRows * vp * sizeof(uint64_t));
    L.total = o;
    return L;
}

// Everything a kernel needs, passed by value.
struct Params {
    const char* logits;
    int64_t row_stride_bytes;
    int32_t dtype, rows, vocab, lp_cols;
    int32_t S;              // slices per row
    int32_t groups;         // row groups of the persistent launch
    int32_t cps;            // chunks per slice
    int32_t epc;            // elements per 16-byte chunk
    int32_t vec_ok;         // rows are 16-byte aligned
    int32_t apply_pen;
    int32_t argmax_only;
    int64_t epoch;
    const float* scale;
    const int32_t* top_k;
    const float* top_p;
    const float* min_p;
    const int32_t* flags;
    const int32_t* logprobs;
    const double* uniform;
    const float* rep;
    const float* pres;
    const float* freq;
    const int64_t* hist_off;
    const int32_t* hist_ids;
    // outputs
    int64_t* tokens;
    int32_t* status;
    uint32_t* tk_key;
    uint64_t* cut_comp;
    float* row_max;
    uint64_t* kept_mass;
    uint64_t* row_mass;
    float* chosen_lp;
    int64_t* top_ids;
    float* top_lp;
    // workspace
    RowState* st;
    PenMeta* pen;
    unsigned long long* wbatch;
    uint32_t* chist;
    uint32_t* mcnt;
    unsigned long long* mmass;
    uint64_t* candA;
    uint64_t* candB;
    int32_t* seg;
    int32_t* pen_ids;
    float* pen_vals;
    uint32_t* pen_cnt;
    uint64_t* fb_keys;
    int64_t fb_pow2;
};

}  // namespace fie
