// The lm_head projection with the sampler's streaming pass as its epilogue.
//
// The reference computes a decode step's logits with the model's output layer,
// an nn.Linear without bias in the model dtype (continuous_batching.py:1345,1594,
// 2225: `self._lm_head()(hidden)`), writes them to a buffer and hands that buffer
// to the sampler (:1926-1928), whose first act is a full read of it.  k_lmhead
// computes logits = hidden · weightᵀ on the matrix cores (bf16 or fp16 operands,
// fp32 accumulation, rounded to nearest-even in the model dtype as the layer's
// output is), writes them once for the passes that need the row again (the
// full-row path, the kept-set check), and runs scan_tile over each 2048-token
// tile it produced: the tile partials k_scan would have read back from HBM.
#pragma once

#include "launchers.h"

namespace fie {

constexpr int kLhRows = 64;                   // rows per workgroup (4 groups of 16)
constexpr int kLhThreads = 512;               // 8 waves: 4 row groups x 2 token groups
constexpr int kLhWaves = kLhThreads / 64;
constexpr int kLhSub = 128;                   // tokens per sub-block (64 per token group)
constexpr int kLhK = 32;                      // K of one MFMA step
constexpr int kLhKStage = 64;                 // K of one pipeline stage (two MFMA steps)
constexpr int kLhStages = 3;                  // LDS stages (two in flight while one is used)
constexpr int kLhRowsPerWave = kLhRows / kLhWaves;
// One stage in 16-byte chunks: A 64 rows x 8, then B 128 tokens x 8; three per thread.
constexpr int kLhChunksA = kLhRows * (kLhKStage / 8);
constexpr int kLhChunks = kLhChunksA + kLhSub * (kLhKStage / 8);
static_assert(kLhChunks == 3 * kLhThreads, "three chunks per thread per stage");
static_assert(kLhKStage / kLhK == 2, "the fragment wait names two MFMA steps' operands");

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// D += A (16 x 32) B (32 x 16).  Lane l supplies A's row l % 16 and B's column
// l % 16, eight consecutive k each from k-group l / 16; it receives D rows
// 4 (l / 16) .. +3 of column l % 16.  A and B take their k the same way, so the
// order the instruction pairs k in does not change the sum's terms.
template <int DT>
FIE_DEV f32x4_t mfma_16x16x32(u32x4_t a, u32x4_t b, f32x4_t c)
{
    if constexpr (DT == FIE_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                      __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// fp32 to the logits dtype, round to nearest even (NaN stays NaN).
template <int DT>
FIE_DEV uint16_t round_logit(float v)
{
    if constexpr (DT == FIE_BF16) {
        uint32_t b = __float_as_uint(v);
        if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((b >> 16) | 0x40u);
        b += 0x7FFFu + ((b >> 16) & 1u);
        return (uint16_t)(b >> 16);
    } else {
        const _Float16 h = (_Float16)v;
        return __builtin_bit_cast(uint16_t, h);
    }
}

// LDS: the GEMM's operand stages, then (reusing the space) the epilogue's
// per-wave penalty counts and marks of one row's tile and the candidate staging
// of scan_tile.
template <bool LONGH>
struct LhEpi {
    uint32_t cnt[kLhWaves][LONGH ? kTile : kTile / 2];
    uint32_t pbits[kLhWaves][kTile / 32];
    uint64_t stage[kLhWaves][kStageW];
    uint32_t uniq[kLhWaves];
};
template <bool LONGH>
union LhSmem {
    uint4 ops[kLhStages][kLhChunks];
    LhEpi<LONGH> e;
};

typedef __attribute__((address_space(3))) void lds_void_t;

// s_waitcnt with vmcnt = n (n < 64) and no wait on the other counters.
constexpr int vmcnt_imm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }

// 16 bytes of LDS at byte address `addr`, read by an instruction the compiler does
// not track: its wait placement would otherwise drain every outstanding copy
// into LDS before any LDS read.  The caller waits on lgkmcnt before use.
FIE_DEV u32x4_t lds_read16(uint32_t addr)
{
    u32x4_t r;
    asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(addr) : "memory");
    return r;
}

FIE_DEV uint32_t lds_addr(const void* p)
{
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Chunk c (of 8) of operand row n sits at slot n * 8 + (c ^ (n & 7)): the eight
// lanes one LDS cycle serves read eight rows' chunk c from eight distinct bank groups.
FIE_DEV int lh_slot(int n, int c) { return n * 8 + (c ^ (n & 7)); }

// Grid: 8 * ceil(NT / 8) * nrb workgroups.  Workgroups are dealt to the eight
// XCDs round robin, so b, b + 8, b + 16, ... share one XCD; there, the nrb row
// blocks of a tile come one after another and read the tile's weight rows
// through that XCD's L2.
template <int DT, bool VEC, bool LONGH>
__global__ __launch_bounds__(kLhThreads, 4) void k_lmhead(const KParams P, const uint16_t* __restrict__ hid,
                                                       const uint16_t* __restrict__ wt, int H, int nrb)
{
    constexpr int EPL = DTy<DT>::EPL, NL = kEPT / EPL;
    __shared__ LhSmem<LONGH> L;
    const fie_sampler_args& a = P.a;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int B = a.rows, V = a.vocab, NT = P.NT;
    const int xcd = blockIdx.x & 7, k = blockIdx.x >> 3;
    const int tile = 8 * (k / nrb) + xcd, rb = k % nrb;
    if (tile >= NT) return;
    if (blockIdx.x == 0 && tid < 2) P.w.dq[tid] = 0u;   // k_deep's queue, filled by k_finish
    if (P.helpers && blockIdx.x == 0 && tid < B) P.w.harr[tid] = 0u;   // k_finish's arrivals
    const int r0 = rb * kLhRows;
    const int64_t ld = a.row_stride;
    uint16_t* out = (uint16_t*)a.logits;

    // 1. The GEMM, 128 tokens of the tile at a time (16 sub-blocks), K in stages of
    //    64 through a three-stage LDS pipeline filled by direct global-to-LDS copies
    //    (two stages in flight while one is read); one barrier per stage, no fence,
    //    so the waits on the copies stay partial.  Wave (rg, tg) computes rows
    //    r0 + 16 rg .. +15 by tokens 64 tg .. +63 of the sub-block.
    const int rg = wv & 3, tg = wv >> 2;
    const int nk = H / kLhKStage;
    const int nsteps = (kTile / kLhSub) * nk;
    // the copies this thread makes, one per 16-byte chunk: slots tid, tid + 512, tid + 1024
    const uint16_t* src[3];
    int sk[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const int p = j * kLhThreads + tid;
        const bool isa = p < kLhChunksA;
        const int pp = isa ? p : p - kLhChunksA;
        const int n = pp >> 3, c = (pp & 7) ^ (n & 7);
        sk[j] = c * 8;
        if (isa) {
            const int row = r0 + n;
            src[j] = hid + (size_t)(row < B ? row : 0) * H;
        } else {
            src[j] = nullptr;      // weight rows depend on the sub-block: set per copy
            sk[j] |= n << 16;      // remember the token within the sub-block
        }
    }
    auto issue = [&](int g) {
        // the stage buffer follows g; past the end the source re-reads the start (unused)
        lds_void_t* base = (lds_void_t*)&L.ops[g % kLhStages][0];
        g = g < nsteps ? g : g - nsteps;
        const int sb = g / nk, k0 = (g - sb * nk) * kLhKStage;
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const uint16_t* gp;
            if (j == 0) {
                gp = src[0] + k0 + sk[0];
            } else {
                const int tok = tile * kTile + sb * kLhSub + (sk[j] >> 16);
                gp = wt + (size_t)(tok < V ? tok : 0) * H + k0 + (sk[j] & 0xFFFF);
            }
            __builtin_amdgcn_global_load_lds((const void*)gp,
                                             (lds_void_t*)((__attribute__((address_space(3))) char*)base +
                                                           (j * kLhThreads + wv * 64) * 16),
                                             16, 0, 0);
        }
    };
    issue(0);
    issue(1);
    f32x4_t acc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    const int an = rg * 16 + (lane & 15);
    for (int g = 0; g < nsteps; ++g) {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(3));     // stage g has landed (g + 1 may not)
        __builtin_amdgcn_s_barrier();
        const uint32_t st = lds_addr(&L.ops[g % kLhStages][0]);
        u32x4_t fa[kLhKStage / kLhK], fb[kLhKStage / kLhK][4];
#pragma unroll
        for (int kk = 0; kk < kLhKStage / kLhK; ++kk) {
            const int c = kk * 4 + (lane >> 4);
            fa[kk] = lds_read16(st + 16u * (uint32_t)lh_slot(an, c));
#pragma unroll
            for (int q = 0; q < 4; ++q)
                fb[kk][q] = lds_read16(st + 16u * (uint32_t)(kLhChunksA + lh_slot(tg * 64 + q * 16 + (lane & 15), c)));
        }
        // the wait names the fragments, so no use of them can be scheduled above it
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(fa[0]), "+v"(fa[1]), "+v"(fb[0][0]), "+v"(fb[0][1]), "+v"(fb[0][2]),
                       "+v"(fb[0][3]), "+v"(fb[1][0]), "+v"(fb[1][1]), "+v"(fb[1][2]), "+v"(fb[1][3])
                     :
                     : "memory");
#pragma unroll
        for (int kk = 0; kk < kLhKStage / kLhK; ++kk) {
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[q] = mfma_16x16x32<DT>(fa[kk], fb[kk][q], acc[q]);
        }
        // a finished sub-block's logits are stored before the next copies: stores
        // count in vmcnt too, and issued first they cannot keep vmcnt(3) from
        // meaning "the next stage has landed" (loads complete in issue order)
        const int sb = g / nk;
        if (g - sb * nk == nk - 1) {
            const int n0 = tile * kTile + sb * kLhSub + tg * 64;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int tok = n0 + q * 16 + (lane & 15);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = r0 + rg * 16 + (lane >> 4) * 4 + i;
                    if (row < B && tok < V) out[(size_t)row * ld + tok] = round_logit<DT>(acc[q][i]);
                }
                acc[q] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
        issue(g + 2);
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));          // the copies past the end, before the space is reused
    // every logit of the workgroup's tile is written before any wave reads it back
    __threadfence();
    __syncthreads();

    // 2. The epilogue: each wave takes 8 rows through scan_tile (k_scan's steps 3-6)
    //    on the tile just written, which is still in this XCD's L2.  The penalty
    //    counts come from k_prep's span bucket, as in k_scan, for this tile only.
    const int lo = tile * kTile;
    const int sp = tile / kWavesPerWG;
    const uint32_t toff = (uint32_t)(lo - sp * kSpan);
    uint32_t* cnt = L.e.cnt[wv];
    uint32_t* pbits = L.e.pbits[wv];
    for (int q = 0; q < kLhRowsPerWave; ++q) {
        const int row = r0 + wv * kLhRowsPerWave + q;
        if (row >= B) break;                                 // uniform in the wave
        const RowCfg rc = row_cfg(a, row);
        const size_t slot = (size_t)row * NT + tile;
        const char* rowp = (const char*)a.logits + (size_t)row * (size_t)ld * 2;
        uint4 raw[NL];
#pragma unroll
        for (int j = 0; j < NL; ++j) raw[j] = load_group<DT, VEC>(rowp, lo + (j * 64 + lane) * EPL, V);
        if (rc.pen) {
            for (int i = lane; i < (LONGH ? kTile : kTile / 2); i += 64) cnt[i] = 0;
            for (int i = lane; i < kTile / 32; i += 64) pbits[i] = 0;
            if (lane == 0) L.e.uniq[wv] = 0;
            wave_lds_sync();
            auto count = [&](uint32_t o) {
                uint32_t was;
                if (LONGH) {
                    was = atomicAdd(&cnt[o], 1u);
                } else {
                    const uint32_t sh = (o & 1) * 16;
                    was = (atomicAdd(&cnt[o >> 1], 1u << sh) >> sh) & 0xFFFFu;
                }
                if (was == 0) {
                    atomicOr(&pbits[o >> 5], 1u << (o & 31));
                    atomicAdd(&L.e.uniq[wv], 1u);
                }
            };
            const size_t rs = (size_t)row * P.NS + sp;
            const uint32_t nb = P.w.nb[rs];
            if (nb <= (uint32_t)kBucketCap) {
                for (uint32_t i = lane; i < nb; i += 64) {
                    const uint32_t o = (uint32_t)P.w.bk[rs * kBucketCap + i] - toff;
                    if (o < (uint32_t)kTile) count(o);
                }
            } else {
                const int64_t h0 = a.hist_offsets[row], h1 = hist_end(a, row);
                for (int64_t h = h0 + lane; h < h1; h += 64) {
                    const uint32_t id = (uint32_t)a.hist_ids[h];
                    const uint32_t o = id - (uint32_t)lo;
                    if (id != 0 && id < (uint32_t)V && o < (uint32_t)kTile) count(o);
                }
            }
            wave_lds_sync();
            if (lane == 0) P.w.nu[slot] = L.e.uniq[wv];
        } else if (lane == 0) {
            P.w.nu[slot] = 0;
        }
        scan_tile<DT, LONGH>(P, rc, row, tile, raw, rowp, pbits, cnt, lo, L.e.stage[wv]);
        wave_lds_sync();
    }
}

}  // namespace fie
