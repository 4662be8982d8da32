// Batched correlation lookup windows from pre-split features (gfx950).
//
// Reference semantics: the volume vol[p][q] = alpha * sum_c fi[c][p] * fj[c][q]
// (cublasGemmBatchedEx, cuda_slam/main.cu:1573-1581), its 2x2 average-pool
// pyramid over the target dims (avg_pool_2x2_kernel, main.cu:1150-1170) and
// the radius-3 lookup that batch_corr_sample_kernel (main.cu:1175-1217) makes
// of every level. The lookup of source pixel p at level l only reads the 8x8
// cells from (floor(x*2^-l) - 3, floor(y*2^-l) - 3); those windows are all this
// path produces, into [slot][4 levels][8 rows][HW][8] (k_corr_lookup_win then
// weights them into the 196 output channels).
//
// Pooling is linear in the target, so level l of the pyramid is the product of
// the source features with the pooled target features:
//     pool_l(vol)[p][q] = alpha * fi[:,p] . pool_l(fj)[:,q]
// Every level is therefore one GEMM over a concatenated target set (level-0
// pixels, then level 1, 2, 3: HW + HW/4 + ... rows), with no pooling of the
// product at all. This re-associates the reference's fp32 sums (the pyramid
// cells agree to fp32 rounding, ~1e-7 relative); with integer-coded features
// every intermediate is exact and the windows are bitwise equal.
//
// Stage 0 (k_frame_max, fp16 split only): partial maxima of |x| over each
// frame's level-0 features (a pooled value is an average, never larger).
// Stage 1 (k_feat_prep), once per frame a launch uses: the fp32 pooled
// features of levels 1..3 (formed in LDS from level 0) and a hi/lo split of
// every pixel of all levels, stored chunk-major [plane][C/16][rows][16] so a
// 16-channel chunk of consecutive rows is one contiguous block, followed by
// one float per frame: the inverse of the frame's split scale.
//   fp16 split (SLK_PREC_F16X3, the default): a frame's features are scaled
//   by one power of two 2^e chosen from the frame's largest magnitude m
//   (m * 2^e in [2^14, 2^15)), then hi = rne_f16(x 2^e),
//   lo = rne_f16(x 2^e - hi): 22 significant bits relative to m, the
//   dropped lo.lo term ~2^-22 m^2 per product. fp16 features are taken with
//   e >= 0, which makes hi exact and lo zero at level 0.
//   bf16 split (SLK_PREC_BF16X3): hi = rne_bf16(x), lo = rne_bf16(x - hi),
//   no scale (16 significant bits, lo.lo ~2^-16).
// Stage 2 (tile_mask_edge, workgroups of the same launch as stage 1): which
// (edge, source tile, target tile) pairs hold any window cell; the others are
// never computed.
// Stage 3 (k_corr_split_win): a workgroup computes 128 sources x 256 targets as
// hi.hi + hi.lo + lo.hi on v_mfma_f32_32x32x16_f16 (or _bf16) (exact
// products, fp32 accumulation), staging 16-channel chunks through LDS in a
// 3-stage ring filled by direct-to-LDS loads, so the loads of chunk k+2 are in
// flight during the MFMAs of chunk k. A pass whose operand plane is zero is
// not issued: with fp16 features every level-0 lo is zero, so a level-0 tile
// takes the one pass hi.hi (the reference's fp16 x fp16 -> fp32 products,
// main.cu:1573-1581) and a pooled tile hi.hi + hi.lo. The accumulator tile
// is then transposed through LDS ([target][source]) and the window cells that
// fall inside the tile are read back with one lane per (source, window
// column), walking the 8 window rows: each masked store covers one row of 8
// sources' windows, multiplied by alpha times both frames' inverse scales
// (powers of two: the scaling adds no rounding). Only ~2% of the level-0 products are
// window cells, and none of them costs more than its LDS round trip.
#include <algorithm>
#include <climits>
#include <type_traits>

#include "corr_common.hpp"

namespace slk {
namespace {

constexpr int kSrcTile = 128;  // sources per workgroup
constexpr int kTgtTile = 256;  // targets per workgroup
constexpr int kChunk = 16;     // channels per LDS stage
constexpr int kStages = 3;     // LDS stages: chunk k+2 streams in while chunk k is used
// word 3 of a raw buffer resource on gfx9-family parts (32-bit data format,
// no swizzle; range checking against num_records)
constexpr int kBufWord3 = 0x00020000;
// an offset past any buffer this file builds a resource for: such a store is
// discarded by the range check
constexpr int kBufDiscard = 0x7FFFFFF0;
constexpr int kTStride = 68;   // floats per transposed-tile row (64 sources + 4 pad)
constexpr int kMaxSlots = 2 * kMaxEdgesPerLaunch;

struct Geom {
    int HW, Ttot, C, levels;
    int off[kMaxLevels];   // first row of level l in the concatenated target set
    int h[kMaxLevels], w[kMaxLevels];
};

// Frame of each feature slot: a host-built list, or (device edge indices)
// slot s < nb -> da[s], else db[s - nb].
struct SlotFrames {
    const int* da;
    const int* db;
    int nb;
    int ident;  // slot s holds frame s (prepared frames)
    int f[kMaxSlots];
};

struct EdgeSlots {
    int si[kMaxEdgesPerLaunch];  // source slot of edge e
    int sj[kMaxEdgesPerLaunch];  // target slot of edge e
};

__device__ __forceinline__ int slot_frame(const SlotFrames& m, int s) {
    if (m.ident) return s;
    if (m.da) return s < m.nb ? m.da[s] : m.db[s - m.nb];
    return m.f[s];
}

__device__ __forceinline__ float ldf(const float* p) { return *p; }
__device__ __forceinline__ float ldf(const _Float16* p) { return (float)(*p); }
// four consecutive elements (16 or 8 bytes, aligned to that size)
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ldf4(const float* p) {
    return *reinterpret_cast<const float4*>(p);
}
__device__ __forceinline__ float4 ldf4(const _Float16* p) {
    const half4_t h = *reinterpret_cast<const half4_t*>(p);
    return make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
}

// Which (edge, source tile, target tile) pairs hold at least one window cell:
// per source and level present, the window's clipped rows/columns span the
// concatenated target indices [off + ya*w + xa, off + yb*w + xb], and every
// target tile in that span is marked (a superset of the tiles holding a cell).
// Tiles not marked are skipped by k_corr_split_win: they would store nothing.
// One workgroup (kT threads, 512 or 1024) per edge: an LDS bitmap (`bits`, at least
// ceil(mtiles * ntiles / 32) words; in the level-1 array when it fits there,
// the sort's histograms then taking the level-0 array, else in the level-0
// array with the sources left in pixel order) of the edge's tiles, then the marked ones
// compacted in tile order into the edge's segment list[e * tpe ..] (ids
// mt * ntiles + nt) and their number into ctr[kCtrCount + e]. Edge 0 also
// zeroes the tile counters of k_corr_split_win, which runs after this on the
// same stream. These workgroups run in the launch of k_feat_prep, beside the
// feature preparation they do not depend on.
// (k_feat_prep launches with kT = 512 or 1024 threads a workgroup; the
// tile-mask chain of an edge then sorts with kT / 64 waves.)
// the preparation's level-0 block (16 channels of 8 x 64 pixels) in LDS,
// which a tile-mask workgroup uses for its sort's histograms or its bitmap
constexpr int kPrepRows = 8, kPrepCols = 64;
constexpr int kPrepLdsWords = kChunk * kPrepRows * kPrepCols;
constexpr int kCtrXcd = 0;     // [0..7] next list index of each XCD's eighth
constexpr int kCtrCount = 8;   // [8..8+edges) marked tiles of each edge
constexpr int kCtrInts = kCtrCount + kMaxEdgesPerLaunch;
struct MaskArgs {
    const float* coords;
    int* list;
    int* ctr;
    int* order;  // [edge][3][HW]: pixel, x, y of each sorted source position
    int mtiles, ntiles, nedges;
    const unsigned long long* tab;  // window_tiles by floored coordinates, or null
};

// Target tiles holding a cell of the 8x8 windows (every level) of a source
// whose coordinates floor to (fx, fy), as bits t of a 64-bit mask for target
// tile t (ntiles <= 64).
__device__ __forceinline__ unsigned long long window_tiles(const Geom& g, int fx, int fy) {
    unsigned long long m = 0ull;
    for (int l = 0; l < g.levels; l++) {
        const int ox = (fx >> l) - 3, oy = (fy >> l) - 3;
        const int xa = std::max(ox, 0), xb = std::min(ox + 7, g.w[l] - 1);
        const int ya = std::max(oy, 0), yb = std::min(oy + 7, g.h[l] - 1);
        if (xa > xb || ya > yb) continue;
        const int lo = (g.off[l] + ya * g.w[l] + xa) / kTgtTile;
        const int hi = (g.off[l] + yb * g.w[l] + xb) / kTgtTile;
        m |= (hi == 63 ? 0ull : (2ull << hi)) - (1ull << lo);
    }
    return m;
}

// window_tiles of every floored source position that can reach the image,
// (fx, fy) in [-kTabPad, w + kTabPad) x [-kTabPad, h + kTabPad), at entry
// (fy + kTabPad) * (w + 2 kTabPad) + fx + kTabPad. Outside that range no
// level has a window cell: level l's window columns (fx >> l) - 3 ..
// (fx >> l) + 4 meet 0 .. w_l - 1 only for -4 * 2^l <= fx < (w_l + 3) * 2^l,
// inside [-32, w + 24) for l <= 3, and likewise for the rows.
constexpr int kTabPad = 32;

__global__ __launch_bounds__(256) void k_mask_table(Geom g, unsigned long long* tab) {
    const int tw = g.w[0] + 2 * kTabPad, th = g.h[0] + 2 * kTabPad;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= tw * th) return;
    tab[i] = window_tiles(g, i % tw - kTabPad, i / tw - kTabPad);
}

// window_tiles(g, fx, fy), from the table when there is one
__device__ __forceinline__ unsigned long long tile_mask_of(const Geom& g,
                                                           const unsigned long long* tab,
                                                           int fx, int fy) {
    if (!tab) return window_tiles(g, fx, fy);
    const int tw = g.w[0] + 2 * kTabPad, th = g.h[0] + 2 * kTabPad;
    const int tx = fx + kTabPad, ty = fy + kTabPad;
    return (unsigned)tx < (unsigned)tw && (unsigned)ty < (unsigned)th ? tab[ty * tw + tx] : 0ull;
}

// ORs mask m (bit t = tile row + t) into the bitmap; a word is touched only
// when it receives a set bit, so only words of existing tiles are
__device__ __forceinline__ void merge_tiles(unsigned* bits, int row, unsigned long long m) {
    const int w0 = row >> 5, sh = row & 31;
    const unsigned part[2] = {(unsigned)m, (unsigned)(m >> 32)};
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const unsigned a = part[k] << sh, b = sh ? part[k] >> (32 - sh) : 0u;
        if (a) atomicOr(&bits[w0 + k], a);
        if (b) atomicOr(&bits[w0 + k + 1], b);
    }
}

// Marks the target tiles of one source in row `row` of the bitmap (any ntiles)
__device__ __forceinline__ void mark_source(const Geom& g, int fx, int fy, int row, int ntiles,
                                            unsigned* bits, const unsigned long long* tab) {
    if (ntiles <= 64) {
        const unsigned long long m = tile_mask_of(g, tab, fx, fy);
        if (m) merge_tiles(bits, row, m);
        return;
    }
    for (int l = 0; l < g.levels; l++) {
        const int ox = (fx >> l) - 3, oy = (fy >> l) - 3;
        const int xa = std::max(ox, 0), xb = std::min(ox + 7, g.w[l] - 1);
        const int ya = std::max(oy, 0), yb = std::min(oy + 7, g.h[l] - 1);
        if (xa > xb || ya > yb) continue;
        const int lo = (g.off[l] + ya * g.w[l] + xa) / kTgtTile;
        const int hi = (g.off[l] + yb * g.w[l] + xb) / kTgtTile;
        for (int t = row + lo; t <= row + hi; t++) atomicOr(&bits[t >> 5], 1u << (t & 31));
    }
}

// Source order of an edge: its pixels sorted by the first row of their
// level-0 window (floor(y) - 3, clamped to [-8, h]: rows outside never meet
// the image at level 0), stably (pixel order within a row). Source tiles are
// runs of 128 sorted sources, so a tile's windows span few image rows and far
// fewer target tiles hold any of their cells than for 128 sources in image
// order (whose +-8 px flows spread them over ~26 rows). A window cell is the
// same dot product whichever tile computes it, so the order changes which
// products are skipped, not any output. Counting sort in the workgroup:
// every wave takes a contiguous 64/kT of the pixels, 64 at a time, and
// counts their keys in its own LDS histogram (atomic adds: the counts do not
// depend on their order); then bucket-major offsets; then the same chunks
// again in pixel order, the lanes of a chunk holding equal keys finding each
// other by one ballot per key bit: each lane takes its bucket's next slot
// plus its rank among the equal lanes below it (the lowest of them advances
// the slot), writes its pixel and coordinates there, and marks the target
// tiles of its windows in the row of its source tile (masks formed in the
// histogram pass when a wave's pixels stay in registers). Writes ord[0][q] =
// the pixel at sorted position q and ord[1][q], ord[2][q] = its x, y. `lds` holds 2 * (kT / 64) * kSortBuckets ints (or is null: no room). A map with
// more rows than that is not sorted: returns false, and neither ord nor the
// bitmap is written.
constexpr int kSortBuckets = 256;

// the lanes of the wave whose key equals this lane's, among `live`
__device__ __forceinline__ unsigned long long equal_keys(int key, int nbits,
                                                         unsigned long long live) {
    unsigned long long m = live;
    for (int b = 0; b < nbits; b++) {  // uniform
        const bool bit = (key >> b) & 1;
        const unsigned long long bal = __ballot(bit);
        m &= bit ? bal : ~bal;
    }
    return m;
}

template <int kT>
__device__ bool sort_and_mark(const Geom& g, const float* cc, int* ord, int* lds, int* wsum,
                              unsigned* bits, int ntiles, const unsigned long long* tab) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int HW = g.HW, nb = g.h[0] + 9;
    if (nb > kSortBuckets || !lds) return false;
    float* oxy = reinterpret_cast<float*>(ord + HW);
    const int nbits = 32 - __builtin_clz(nb - 1);
    const unsigned long long below = (1ull << lane) - 1ull;
    int* hist = lds;                             // [(kT / 64)][kSortBuckets]
    int* pos = lds + (kT / 64) * kSortBuckets;  // [(kT / 64)][kSortBuckets]: next slot
    for (int i = tid; i < (kT / 64) * kSortBuckets; i += kT) hist[i] = 0;
    __syncthreads();  // also orders the caller's clearing of the bitmap
    const int part = (HW + (kT / 64) - 1) / (kT / 64);  // pixels of each wave
    const int q0 = std::min(HW, wv * part), q1 = std::min(HW, q0 + part);
    auto key_of = [&](float y) {
        const int oy = floor_clamped(y) - 3;
        return std::min(std::max(oy, -8), g.h[0]) + 8;
    };
    // the coordinates of kG chunks are loaded before the first is used; when
    // a wave's pixels are one such group they stay in registers for the
    // scatter. 1024-thread workgroups serve maps up to 4096 pixels, 256 a
    // wave: 4 chunks, which keeps the launch within 64 VGPRs (two
    // workgroups a CU)
    constexpr int kG = kT >= 1024 ? 4 : 12;
    float xv[kG], yv[kG];
    auto load = [&](int pg) {
#pragma unroll
        for (int u = 0; u < kG; u++) {
            const int p = std::min(pg + 64 * u + lane, q1 - 1);
            xv[u] = cc[p];
            yv[u] = cc[HW + p];
        }
    };
    const bool one = q1 - q0 <= 64 * kG;
    // with the wave's pixels in registers and at most 64 target tiles, each
    // source's tile mask is formed here, while the loads of the histogram
    // pass are what the waves wait for, and only merged in the scatter
    const bool pre = one && ntiles <= 64;
    unsigned long long mk[kG];
    for (int pg = q0; pg < q1; pg += 64 * kG) {
        load(pg);
#pragma unroll
        for (int u = 0; u < kG; u++) {
            if (pg + 64 * u + lane < q1) atomicAdd(&hist[wv * kSortBuckets + key_of(yv[u])], 1);
            mk[u] = pre ? tile_mask_of(g, tab, floor_clamped(xv[u]), floor_clamped(yv[u])) : 0ull;
        }
    }
    __syncthreads();
    {
        // thread b < kSortBuckets: bucket b's total, its exclusive prefix over
        // the buckets (a wave scan, then the totals of the waves below), and
        // each wave's first slot in it
        const int bkt = tid;
        const bool bw = tid < kSortBuckets;  // uniform per wave
        int tot = 0, incl = 0;
        if (bw) {
#pragma unroll
            for (int w = 0; w < (kT / 64); w++) tot += hist[w * kSortBuckets + bkt];
            incl = tot;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const int v = __shfl_up(incl, off, 64);
                if (lane >= off) incl += v;
            }
            if (lane == 63) wsum[wv] = incl;
        }
        __syncthreads();
        if (bw) {
            int start = incl - tot;
            for (int w = 0; w < wv; w++) start += wsum[w];
#pragma unroll
            for (int w = 0; w < (kT / 64); w++) {
                pos[w * kSortBuckets + bkt] = start;
                start += hist[w * kSortBuckets + bkt];
            }
        }
    }
    __syncthreads();
    // stable scatter, chunk by chunk in pixel order: every lane reads its
    // bucket's next slot, adds its rank among the equal lanes below it, and
    // the lowest of them advances the slot past all of them
    for (int pg = q0; pg < q1; pg += 64 * kG) {
        if (!one) load(pg);
#pragma unroll
        for (int u = 0; u < kG; u++) {
            const int pb = pg + 64 * u;
            if (pb >= q1) break;  // uniform
            const int p = pb + lane;
            const bool act = p < q1;
            const int key = act ? key_of(yv[u]) : 0;
            const unsigned long long m = equal_keys(key, nbits, __ballot(act));
            const int base = pos[wv * kSortBuckets + key];
            const int rank = __builtin_popcountll(m & below);
            if (act) {
                const int q = base + rank;
                if (rank == 0) pos[wv * kSortBuckets + key] = base + __builtin_popcountll(m);
                ord[q] = p;
                oxy[q] = xv[u];
                oxy[HW + q] = yv[u];
                if (pre) {
                    if (mk[u]) merge_tiles(bits, q / kSrcTile * ntiles, mk[u]);
                } else {
                    mark_source(g, floor_clamped(xv[u]), floor_clamped(yv[u]),
                                q / kSrcTile * ntiles, ntiles, bits, tab);
                }
            }
        }
    }
    return true;
}

template <int kT>
__device__ void tile_mask_edge(const MaskArgs& a, const Geom& g, int e, unsigned* big,
                               unsigned* small, int small_words, int* wave_sum) {
    const float* coords = a.coords;
    int* list = a.list;
    int* ctr = a.ctr;
    const int mtiles = a.mtiles, ntiles = a.ntiles;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int tpe = mtiles * ntiles;
    const int nw = (tpe + 31) / 32;
    // the bitmap in `small` when it fits, the sort's histograms then in
    // `big` (kPrepLdsWords words); else the bitmap in `big` and no sort
    const bool fits = nw <= small_words;
    unsigned* bits = fits ? small : big;
    for (int i = tid; i < nw; i += kT) bits[i] = 0u;
    if (e == 0 && tid < 8) ctr[kCtrXcd + tid] = 0;
    const float* cc = coords + (size_t)e * 2 * g.HW;
    int* ord = a.order + (size_t)e * 3 * g.HW;
    static_assert(2 * (kT / 64) * kSortBuckets <= kPrepLdsWords, "sort LDS");
    int* sort_lds = fits ? reinterpret_cast<int*>(big) : nullptr;
    if (!sort_and_mark<kT>(g, cc, ord, sort_lds, wave_sum, bits, ntiles, a.tab)) {  // uniform
        // pixel order: the order is the identity, written beside the mask.
        // A wave's 64 consecutive sources lie in one source tile (kSrcTile is
        // a multiple of 64). When an edge's target tiles fit a 64-bit mask,
        // each lane builds the mask of the tiles its windows touch, the wave
        // ORs them by shuffles and lane 0 merges the result into the bitmap;
        // otherwise every lane marks its tiles in the bitmap itself.
        __syncthreads();  // the bitmap is clear
        float* oxy = reinterpret_cast<float*>(ord + g.HW);
        constexpr int kU = 4;  // sources per thread whose coordinates load together
        for (int pb = 0; pb < g.HW; pb += kU * kT) {
            float xs[kU], ys[kU];
#pragma unroll
            for (int u = 0; u < kU; u++) {
                const int q = std::min(pb + u * kT + tid, g.HW - 1);
                xs[u] = cc[q];
                ys[u] = cc[g.HW + q];
            }
#pragma unroll
            for (int u = 0; u < kU; u++) {
                const int pw = pb + u * kT + (tid & ~63);  // the wave's first source
                if (pw >= g.HW) break;                                // uniform
                const bool in = pw + lane < g.HW;
                const int row = pw / kSrcTile * ntiles;  // first tile id of the source tile
                const int fx = floor_clamped(xs[u]), fy = floor_clamped(ys[u]);
                if (in) {
                    ord[pw + lane] = pw + lane;
                    oxy[pw + lane] = xs[u];
                    oxy[g.HW + pw + lane] = ys[u];
                }
                if (ntiles > 64) {
                    if (in) mark_source(g, fx, fy, row, ntiles, bits, a.tab);
                    continue;
                }
                const unsigned long long m = in ? tile_mask_of(g, a.tab, fx, fy) : 0ull;
                unsigned m0 = (unsigned)m, m1 = (unsigned)(m >> 32);
#pragma unroll
                for (int off = 32; off >= 1; off >>= 1) {
                    m0 |= __shfl_xor(m0, off, 64);
                    m1 |= __shfl_xor(m1, off, 64);
                }
                if (lane == 0) merge_tiles(bits, row, ((unsigned long long)m1 << 32) | m0);
            }
        }
    }
    __syncthreads();
    // compaction, kT tiles a round: ballot ranks within a wave,
    // wave totals through LDS
    int* seg = list + (size_t)e * tpe;
    int base = 0;
    for (int t0 = 0; t0 < tpe; t0 += kT) {
        const int t = t0 + tid;
        const bool m = t < tpe && ((bits[t >> 5] >> (t & 31)) & 1u);
        const unsigned long long bal = __ballot(m);
        const int rank = __builtin_popcountll(bal & ((1ull << lane) - 1ull));
        if (lane == 0) wave_sum[wv] = __builtin_popcountll(bal);
        __syncthreads();
        int before = 0, all = 0;
#pragma unroll
        for (int q = 0; q < kT / 64; q++) {
            const int v = wave_sum[q];
            before += q < wv ? v : 0;
            all += v;
        }
        if (m) seg[base + before + rank] = t;
        base += all;
        __syncthreads();  // wave_sum is rewritten by the next round
    }
    if (tid == 0) ctr[kCtrCount + e] = base;
}

// Split modes of the preparation and the window kernel
enum { kSplitBF16 = 0, kSplitF16 = 1 };

// hi = rne_f16(x), lo = rne_f16(x - hi), packed as lo << 16 | hi (|x| < 2^15:
// x - hi is exact in fp32, hi never overflows)
__device__ __forceinline__ unsigned split_f16(float x) {
    const _Float16 h = (_Float16)x;
    const _Float16 l = (_Float16)(x - (float)h);
    return (unsigned)__builtin_bit_cast(unsigned short, h) |
           ((unsigned)__builtin_bit_cast(unsigned short, l) << 16);
}

// The exponent e of a frame's fp16 split scale 2^e from its largest magnitude
// m: m * 2^e in [2^14, 2^15), so every scaled feature and its hi stay below
// 2^15 (fp16 holds up to 65504), bounded to [-120, 120] (2^+-e stays a normal
// float; a bound only lowers m * 2^e); 0 for m = 0 or non-finite. `exact`: at
// least 0 (fp16 features: then x 2^e is exact in fp16 and lo is zero).
__device__ __forceinline__ int split_exponent(float m, bool exact) {
    int e = 0;
    if (m > 0.0f && m <= 3.402823466e38f) {
        e = 15 - __builtin_amdgcn_frexp_expf(m);  // m = f 2^k, f in [0.5, 1)
        e = std::min(std::max(e, -120), 120);
        if (exact) e = std::max(e, 0);
    }
    return e;
}

// Partial maxima of |x| over the frames of slots slot_lo.., for the fp16
// split's per-frame scale: workgroup (q, s) reduces chunks q, q + nparts, ..
// of kMaxChunk elements of slot s's C x HW features into part[s][q] (no
// atomics: the preparation reduces the parts of its slot). Each thread's four
// 16-byte loads of a chunk are in flight together. The pooled levels' values
// are means of level-0 values, so the frame's level-0 maximum bounds every
// level.
constexpr int kMaxParts = 256;              // partial maxima per slot, at most
constexpr int kMaxChunk = 256 * 4 * 4;      // elements a workgroup reduces per round
template <typename Tin>
__global__ __launch_bounds__(256) void k_frame_max(const Tin* __restrict__ fm, long fstride,
                                                   SlotFrames sf, int slot_lo, long n, int vec,
                                                   int nparts, float* __restrict__ part) {
    __shared__ float wm[4];
    const int s = slot_lo + blockIdx.y, q = blockIdx.x, tid = threadIdx.x;
    const Tin* src = fm + (long)slot_frame(sf, s) * fstride;
    float m = 0.0f;
    for (long c0 = (long)q * kMaxChunk; c0 < n; c0 += (long)nparts * kMaxChunk) {
        if (vec) {  // uniform: n % 4 == 0, the frames 4-element aligned
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const long i = c0 + 4 * (tid + 256 * u);
                v[u] = i < n ? ldf4(src + i) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                m = fmaxf(fmaxf(m, fabsf(v[u].x)), fabsf(v[u].y));
                m = fmaxf(fmaxf(m, fabsf(v[u].z)), fabsf(v[u].w));
            }
        } else {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) {
                const long i = c0 + tid + 256 * u;
                v[u] = i < n ? ldf(src + i) : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 16; u++) m = fmaxf(m, fabsf(v[u]));
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((tid & 63) == 0) wm[tid >> 6] = m;
    __syncthreads();
    if (tid == 0) part[(size_t)s * kMaxParts + q] = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
}

// Feature preparation of one frame slot, one launch: a workgroup takes a
// 16-channel chunk of an 8 x 64 block of level-0 pixels into LDS, forms its
// 4 x 32, 2 x 16 and 1 x 8 pooled blocks in turn (each pooled value
// 0.25 * (((a + b) + c) + d) of its 2x2 parents, the parents' row first;
// a pooled pixel's parents always lie in the block), and writes the hi/lo
// split of every pixel of the levels present, 16 channels = 32 bytes per
// pixel and plane, into out[slot][plane][C/16][Ttot][16]; under the fp16
// split every value is first scaled by its frame's 2^e (from the partial
// maxima of k_frame_max), and the first workgroup of a slot stores 2^-e
// after the slot's planes. `pooled` = 0 writes level 0 only (source slots).
// One-dimensional grid: first, when mk.list is set, one tile-mask workgroup
// per edge (tile_mask_edge, with the level-0 and level-1 LDS arrays; they are
// the longer chains, so they are dispatched first), then the blocks x C/16 x
// slots preparation workgroups (block fastest).
// (waves per SIMD: two 1024-thread or three 512-thread workgroups a CU)
template <typename Tin, int kT>
__global__ __launch_bounds__(kT, kT >= 1024 ? 8 : 6) void k_feat_prep(
    const Tin* __restrict__ fm, long fstride, SlotFrames sf, int slot_lo,
    unsigned short* __restrict__ out, long slot_elems, Geom g, int pooled, int vec, int nbx,
    int nblk, int nmask, MaskArgs mk, int mode, const float* __restrict__ part, int nparts) {
    __shared__ float l0[kChunk][kPrepRows][kPrepCols];
    __shared__ float l1[kChunk][kPrepRows / 2][kPrepCols / 2];
    __shared__ float l2[kChunk][kPrepRows / 4][kPrepCols / 4];
    __shared__ float l3[kChunk][kPrepRows / 8][kPrepCols / 8];
    __shared__ int wave_sum[kT / 64];
    __shared__ float fscale;  // the frame's 2^e
    if ((int)blockIdx.x < nmask) {  // uniform
        // the tile-mask chains are the launch's long pole: their waves issue
        // ahead of the preparation waves sharing their SIMDs
        __builtin_amdgcn_s_setprio(2);
        tile_mask_edge<kT>(mk, g, blockIdx.x, reinterpret_cast<unsigned*>(&l0[0][0][0]),
                           reinterpret_cast<unsigned*>(&l1[0][0][0]), (int)(sizeof(l1) / 4),
                           wave_sum);
        return;
    }
    const int tid = threadIdx.x;
    const int b = blockIdx.x - nmask;
    const int blk = b % nblk, rest = b / nblk;
    const int bx = blk % nbx, by = blk / nbx;
    const int k = rest % (g.C / kChunk), s = slot_lo + rest / (g.C / kChunk);
    const int W = g.w[0], H = g.h[0];
    const Tin* src = fm + (long)slot_frame(sf, s) * fstride + (long)(k * kChunk) * g.HW;
    if (tid < 64) {  // the frame's scale, from the partial maxima of its slot
        float m = 0.0f;
        if (mode == kSplitF16)
            for (int q = tid; q < nparts; q += 64) m = fmaxf(m, part[(size_t)s * kMaxParts + q]);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
        if (tid == 0)
            fscale = mode == kSplitF16
                         ? __builtin_amdgcn_ldexpf(
                               1.0f, split_exponent(m, std::is_same<Tin, _Float16>::value))
                         : 1.0f;
    }
    // all of a thread's loads are issued before the first is used
    constexpr int kPer = kChunk * kPrepRows * kPrepCols / kT;
    float ld[kPer];
    if (vec) {  // uniform: W % 4 == 0 and the frames 4-element aligned
        // four consecutive pixels of a row a lane (all inside or all outside)
#pragma unroll
        for (int u = 0; u < kPer / 4; u++) {
            const int i = 4 * (tid + u * kT);
            const int c = i / (kPrepRows * kPrepCols);
            const int r = (i / kPrepCols) % kPrepRows, x = i % kPrepCols;
            const int yy = by * kPrepRows + r, xx = bx * kPrepCols + x;
            const bool in = yy < H && xx < W;
            const float4 v = ldf4(src + (in ? (long)c * g.HW + (long)yy * W + xx : 0L));
            ld[4 * u] = in ? v.x : 0.0f;
            ld[4 * u + 1] = in ? v.y : 0.0f;
            ld[4 * u + 2] = in ? v.z : 0.0f;
            ld[4 * u + 3] = in ? v.w : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kPer / 4; u++) {
            const int i = 4 * (tid + u * kT);
            *reinterpret_cast<float4*>(
                &l0[i / (kPrepRows * kPrepCols)][(i / kPrepCols) % kPrepRows][i % kPrepCols]) =
                make_float4(ld[4 * u], ld[4 * u + 1], ld[4 * u + 2], ld[4 * u + 3]);
        }
    } else {
#pragma unroll
        for (int u = 0; u < kPer; u++) {
            const int i = tid + u * kT;
            const int c = i / (kPrepRows * kPrepCols);
            const int r = (i / kPrepCols) % kPrepRows, x = i % kPrepCols;
            const int yy = by * kPrepRows + r, xx = bx * kPrepCols + x;
            const bool in = yy < H && xx < W;
            ld[u] = ldf(src + (in ? (long)c * g.HW + (long)yy * W + xx : 0L));
            if (!in) ld[u] = 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kPer; u++) {
            const int i = tid + u * kT;
            l0[i / (kPrepRows * kPrepCols)][(i / kPrepCols) % kPrepRows][i % kPrepCols] = ld[u];
        }
    }
    __syncthreads();
    const float sc = fscale;
    const size_t plane = (size_t)g.C * g.Ttot;
    unsigned short* const slot = out + (size_t)s * slot_elems;
    if (blk == 0 && k == 0 && tid == 0)  // the slot's inverse scale (a power of two)
        *reinterpret_cast<float*>(slot + 2 * plane) = 1.0f / sc;
    unsigned short* const base = slot + (size_t)k * g.Ttot * kChunk;
    auto emit = [&](int t, const float (&v)[kChunk]) {
        u16x8_t hi[2], lo[2];
#pragma unroll
        for (int u = 0; u < kChunk; u++) {
            const unsigned pk = mode == kSplitF16 ? split_f16(v[u] * sc) : split_bf16(v[u]);
            hi[u >> 3][u & 7] = (unsigned short)(pk & 0xffffu);
            lo[u >> 3][u & 7] = (unsigned short)(pk >> 16);
        }
        unsigned short* o = base + (size_t)t * kChunk;
        *reinterpret_cast<u16x8_t*>(o) = hi[0];
        *reinterpret_cast<u16x8_t*>(o + 8) = hi[1];
        *reinterpret_cast<u16x8_t*>(o + plane) = lo[0];
        *reinterpret_cast<u16x8_t*>(o + plane + 8) = lo[1];
    };
    // level 0
    for (int p = tid; p < kPrepRows * kPrepCols; p += kT) {
        const int r = p / kPrepCols, x = p % kPrepCols;
        const int yy = by * kPrepRows + r, xx = bx * kPrepCols + x;
        if (yy >= H || xx >= W) continue;
        float v[kChunk];
#pragma unroll
        for (int c = 0; c < kChunk; c++) v[c] = l0[c][r][x];
        emit(yy * W + xx, v);
    }
    if (!pooled) return;
    // pooled levels: level l from level l-1 in LDS, then its pixels out
    auto level = [&](auto& dst, const auto& from, int l, int rows, int cols) {
        for (int i = tid; i < kChunk * rows * cols; i += kT) {
            const int c = i / (rows * cols), r = (i / cols) % rows, x = i % cols;
            float sum = from[c][2 * r][2 * x] + from[c][2 * r][2 * x + 1];
            sum = sum + from[c][2 * r + 1][2 * x];
            sum = sum + from[c][2 * r + 1][2 * x + 1];
            dst[c][r][x] = 0.25f * sum;
        }
        __syncthreads();
        for (int p = tid; p < rows * cols; p += kT) {
            const int r = p / cols, x = p % cols;
            const int yy = by * rows + r, xx = bx * cols + x;
            if (yy >= g.h[l] || xx >= g.w[l]) continue;
            float v[kChunk];
#pragma unroll
            for (int c = 0; c < kChunk; c++) v[c] = dst[c][r][x];
            emit(g.off[l] + yy * g.w[l] + xx, v);
        }
    };
    if (g.levels > 1) level(l1, l0, 1, kPrepRows / 2, kPrepCols / 2);
    if (g.levels > 2) level(l2, l1, 2, kPrepRows / 4, kPrepCols / 4);
    if (g.levels > 3) level(l3, l2, 3, kPrepRows / 8, kPrepCols / 8);
}

struct alignas(16) SplitSmem {
    union {
        struct {
            // [stage][hi/lo][row * 16 + swizzled k]: 32-byte rows, the two
            // 16-byte halves of row r swapped when bit 2 xor bit 3 of r is
            // set, so that the MFMA operand reads (16 lanes = 16 rows per
            // 256-byte pass of a 128-bit read over 64 banks) touch 64
            // distinct banks; the staging writes are contiguous 1 KB blocks
            unsigned short A[kStages][2][kSrcTile * kChunk];
            unsigned short B[kStages][2][kTgtTile * kChunk];
        } st;
        float T[kTgtTile][kTStride];  // [target][source] of one 64-source half
    } u;
    int org[kSrcTile][2];     // floor_clamped(x), floor_clamped(y) of each source
    float crd[2][kSrcTile];   // x, y coordinates of the tile's sources
    int pix[kSrcTile];        // pixel of each source
};

// One direct-to-LDS load per lane (16 or 4 bytes): lane l reads p and writes
// LDS bytes m0 + size*l (m0 = the wave's region). As inline assembly the
// compiler does not track these LDS writes, so it inserts no waits for them
// before the LDS accesses it cannot prove disjoint (which, in the tile loop,
// would mean waiting for every chunk in flight). Every read of staged data is
// ordered by the explicit vmcnt waits and barriers of the chunk loop.
__device__ __forceinline__ void dma_x4(const void* p, unsigned lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(p), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void dma_x1(const void* p, unsigned lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(p), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ unsigned lds_addr(const void* p) { return (unsigned)(size_t)p; }

// s_waitcnt immediates (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8): vmcnt(n) lgkmcnt(0) is 0x0070 | n for n < 16; vmcnt(0)
// lgkmcnt(0), and lgkmcnt(0) alone
constexpr int kWaitVm0Lgkm0 = 0x0070;
constexpr int kWaitLgkm0 = 0xC07F;

// Workgroup barrier for LDS hand-offs only: this wave's LDS accesses are
// complete, but its global stores may still be in flight (__syncthreads'
// fence would wait for those too).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// one 32x32x16 MFMA of the split mode's operand type
template <bool kF16>
__device__ __forceinline__ f32x16 mfma_split(u16x8_t a, u16x8_t b, f32x16 c) {
    if constexpr (kF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                      __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0,
                                                       0);
}

template <bool B>
using bool_c = std::integral_constant<bool, B>;

// Grid: a fixed number of workgroups of 256 threads, two per CU, each taking
// marked tiles (tile_mask_edge) one at a time from its XCD's counter: tile
// index idx runs over the edges' segments concatenated, workgroup blockIdx % 8
// runs on that XCD and serves the XCD's contiguous eighth of those indices,
// so the edges an XCD works on stay in its L2, and no CU idles while tiles
// remain. Waves form a 2x2 grid: wave (wm, wn) owns sources
// wm*64..+63 and targets wn*128..+127 of a tile, eight 32x32 accumulator
// blocks. Source tile mt holds sorted positions mt*128..+127 of the edge's
// order (tile_mask_edge): the A rows are gathered through the order's pixel
// column, the coordinates come from its sorted copies, and each source's
// windows are stored at its own pixel. kF16: fp16 operands (the scaled fp16
// split), else bf16. alo = 0: every source lo is zero (fp16 features, fp16
// split), and so is every level-0 target lo: a tile of level-0 targets then
// takes the one pass hi.hi, a tile with pooled targets hi.hi + hi.lo.
template <bool kF16>
__global__ __launch_bounds__(256, 2) void k_corr_split_win(
    const unsigned short* __restrict__ feat, long slot_elems, EdgeSlots es,
    const int* __restrict__ order, float* __restrict__ win, int slot0, Geom g, float alpha,
    int mtiles, int ntiles, int nedges, const int* __restrict__ list, int* __restrict__ ctr,
    int alo) {
    __shared__ SplitSmem sm;
    __shared__ int next_tile;
    const int tpe = mtiles * ntiles;
    // lane e of every wave holds pre = the number of marked tiles of the
    // edges before e (nedges <= 64); cnt = all of them
    int pre, cnt;
    {
        const int ln = threadIdx.x & 63;
        const int c = ln < nedges ? ctr[kCtrCount + ln] : 0;
        int incl = c;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int v = __shfl_up(incl, off, 64);
            if (ln >= off) incl += v;
        }
        pre = incl - c;
        cnt = __builtin_amdgcn_readlane(incl, 63);
    }
    // Workgroups b and b + gridDim.x / 2 are dispatched to the same CU. Started
    // together they run their chunk loops together and then both extract,
    // leaving the matrix cores idle; the second half starts about half a tile
    // later (three sleeps of 64 x 64 clocks), when there are enough tiles for
    // the offset to pay for itself.
    if (blockIdx.x >= gridDim.x / 2 && cnt >= 4 * (int)gridDim.x) {
        __builtin_amdgcn_s_sleep(64);
        __builtin_amdgcn_s_sleep(64);
        __builtin_amdgcn_s_sleep(64);
    }
    const int xcd = blockIdx.x & 7;
    const int lo = (int)((long long)cnt * xcd / 8), hi = (int)((long long)cnt * (xcd + 1) / 8);
    // The next tile's index is taken at the start of a tile and published in
    // LDS after the chunk loop (whose last wait covers the atomic's return).
    int* const counter = ctr + kCtrXcd + xcd;
    if (threadIdx.x == 0) next_tile = lo + atomicAdd(counter, 1);
    lds_barrier();
    for (int idx = __builtin_amdgcn_readfirstlane(next_tile); idx < hi;
         idx = __builtin_amdgcn_readfirstlane(next_tile)) {  // uniform
    int taken;  // thread 0 only
    if (threadIdx.x == 0) taken = atomicAdd(counter, 1);
    // the edge of tile idx: the last lane whose prefix is <= idx (edges
    // with no marked tile share their successor's prefix)
    const bool before_idx = (int)(threadIdx.x & 63) < nedges && pre <= idx;
    const int e = __builtin_popcountll(__ballot(before_idx)) - 1;
    const int r = list[(size_t)e * tpe + (idx - __builtin_amdgcn_readlane(pre, e))];
    const int mt = r / ntiles, nt = r - mt * ntiles;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    const int HW = g.HW, Ttot = g.Ttot;
    const int p0 = mt * kSrcTile, t0 = nt * kTgtTile;
    const size_t plane = (size_t)g.C * Ttot;
    const unsigned short* fa = feat + (size_t)es.si[e] * slot_elems;
    const unsigned short* fb = feat + (size_t)es.sj[e] * slot_elems;
    // alpha over both frames' split scales (powers of two: no rounding)
    const float fs = alpha * *reinterpret_cast<const float*>(fa + 2 * plane) *
                     *reinterpret_cast<const float*>(fb + 2 * plane);
    const int* ord = order + (size_t)e * 3 * HW;

    // Staging by direct-to-LDS loads (global_load_lds_dwordx4): lane l of wave
    // w writes bytes 16*(64w + l) of a 4 KB region, i.e. row tid/2, physical
    // half tid%2 of the 32-byte-row layout, so each thread loads the logical
    // half that lands there. Rows past the source/target range read a clamped
    // in-range row: an MFMA output D[i][j] only combines row i of A with
    // column j of B, so such rows only reach accumulator cells never read.
    const int hr = tid >> 1;
    const int hh = ((tid & 1) ^ (((hr >> 2) ^ (hr >> 3)) & 1)) * 8;  // rows hr, 128 + hr alike
    // pixel of source row hr (clamped: the DMA below must stay in the frame
    // whatever the order buffer holds)
    const int pa = std::min((unsigned)ord[std::min(p0 + hr, HW - 1)], (unsigned)(HW - 1));
    if (!(tid & 1)) sm.pix[hr] = pa;  // read after the chunk loop's barriers
    const unsigned short* ga = fa + (size_t)pa * kChunk + hh;
    const unsigned short* gb0 = fb + (size_t)std::min(t0 + hr, Ttot - 1) * kChunk + hh;
    const unsigned short* gb1 = fb + (size_t)std::min(t0 + 128 + hr, Ttot - 1) * kChunk + hh;
    const size_t kstep = (size_t)Ttot * kChunk;
    const int wdst = wave * 512;  // this wave's 1 KB of a 4 KB region, in u16

    f32x16 acc[2][4];
#pragma unroll
    for (int sb = 0; sb < 2; sb++)
#pragma unroll
        for (int tb = 0; tb < 4; tb++) acc[sb][tb] = (f32x16){0};
    // MFMA operand layout: lane l holds row l%32, k = 8*(l/32)..+7; every
    // operand block starts at a multiple of 32 rows, so the swizzle bit of the
    // lane's row is bit 2 xor bit 3 of l%32
    const int orow = lane & 31;
    const int ooff = orow * kChunk + ((((lane >> 5) ^ (((orow >> 2) ^ (orow >> 3)) & 1))) * 8);
    const int nk = g.C / kChunk;
    // The chunk loop of one tile, with (kA) or without the source lo plane
    // and (kB) with or without the target lo plane: a plane that is zero is
    // neither staged nor multiplied.
    auto chunk_loop = [&](auto a_lo, auto b_lo) {
        constexpr bool kA = decltype(a_lo)::value, kB = decltype(b_lo)::value;
        constexpr int kLoads = 3 + (kA ? 1 : 0) + (kB ? 2 : 0);  // loads per chunk and thread
        auto issue = [&](int k, int st) {
            const size_t o = (size_t)k * kstep;
            dma_x4(ga + o, lds_addr(&sm.u.st.A[st][0][wdst]));
            if constexpr (kA) dma_x4(ga + plane + o, lds_addr(&sm.u.st.A[st][1][wdst]));
            dma_x4(gb0 + o, lds_addr(&sm.u.st.B[st][0][wdst]));
            dma_x4(gb1 + o, lds_addr(&sm.u.st.B[st][0][2048 + wdst]));
            if constexpr (kB) {
                dma_x4(gb0 + plane + o, lds_addr(&sm.u.st.B[st][1][wdst]));
                dma_x4(gb1 + plane + o, lds_addr(&sm.u.st.B[st][1][2048 + wdst]));
            }
        };
        auto compute = [&](int st) {
            // every operand read of the step goes out first, in the order the
            // MFMAs use them, so the matrix cores wait for the first reads
            // only; each accumulator takes lo.hi, hi.lo, then hi.hi (the small
            // cross terms before the large one)
            u16x8_t ah[2], al[2], bh[4], bl[4];
            if constexpr (kA)
#pragma unroll
                for (int sb = 0; sb < 2; sb++)
                    al[sb] = *reinterpret_cast<const u16x8_t*>(
                        &sm.u.st.A[st][1][(wm * 64 + sb * 32) * kChunk + ooff]);
#pragma unroll
            for (int tb = 0; tb < 4; tb++)
                bh[tb] = *reinterpret_cast<const u16x8_t*>(
                    &sm.u.st.B[st][0][(wn * 128 + tb * 32) * kChunk + ooff]);
#pragma unroll
            for (int sb = 0; sb < 2; sb++)
                ah[sb] = *reinterpret_cast<const u16x8_t*>(
                    &sm.u.st.A[st][0][(wm * 64 + sb * 32) * kChunk + ooff]);
            if constexpr (kB)
#pragma unroll
                for (int tb = 0; tb < 4; tb++)
                    bl[tb] = *reinterpret_cast<const u16x8_t*>(
                        &sm.u.st.B[st][1][(wn * 128 + tb * 32) * kChunk + ooff]);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (kA)
#pragma unroll
                for (int tb = 0; tb < 4; tb++)
#pragma unroll
                    for (int sb = 0; sb < 2; sb++)
                        acc[sb][tb] = mfma_split<kF16>(al[sb], bh[tb], acc[sb][tb]);
            if constexpr (kB)
#pragma unroll
                for (int tb = 0; tb < 4; tb++)
#pragma unroll
                    for (int sb = 0; sb < 2; sb++)
                        acc[sb][tb] = mfma_split<kF16>(ah[sb], bl[tb], acc[sb][tb]);
#pragma unroll
            for (int tb = 0; tb < 4; tb++)
#pragma unroll
                for (int sb = 0; sb < 2; sb++)
                    acc[sb][tb] = mfma_split<kF16>(ah[sb], bh[tb], acc[sb][tb]);
        };

        // Pipeline: at step k the loads of chunks k and k+1 are in flight;
        // wait for this thread's chunk k (kLoads loads) and for every wave at
        // the barrier -- after which chunk k is in LDS and stage (k+2)%3,
        // last read at step k-1, is free for chunk k+2. The wait and barrier
        // are explicit because a workgroup fence would also wait for chunk
        // k+1.
        issue(0, 0);
        // coordinates of the tile's sources, in flight with the first chunk
        // (also by a direct-to-LDS load: every load the pipeline waits on with
        // vmcnt is of the same kind, and those complete in issue order)
        {
            const int half = wave & 1, comp = wave >> 1;  // wave -> sources half*64.., x or y
            const int pc = std::min(p0 + half * 64 + lane, HW - 1);
            dma_x1(ord + (size_t)(1 + comp) * HW + pc, lds_addr(&sm.crd[comp][half * 64]));
        }
        if (nk > 1) issue(1, 1);
        // While in its chunk loop a wave issues at raised priority, so that on
        // a SIMD shared with the other workgroup's extracting wave the MFMA
        // issue goes first and the extraction takes the slots left over.
        __builtin_amdgcn_s_setprio(1);
        for (int k = 0; k < nk; k++) {
            if (k + 1 < nk)
                __builtin_amdgcn_s_waitcnt(kWaitVm0Lgkm0 | kLoads);  // vmcnt(kLoads) lgkmcnt(0)
            else
                __builtin_amdgcn_s_waitcnt(kWaitVm0Lgkm0);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_barrier();
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            if (k + 2 < nk) issue(k + 2, (k + 2) % kStages);
            compute(k % kStages);
        }
    };
    if constexpr (kF16) {
        // a target tile with a pooled row has lo planes (pooled fp16 values
        // are fp32 sums)
        const bool blo = alo || (g.levels > 1 && t0 + kTgtTile > g.off[1]);
        if (alo)
            chunk_loop(bool_c<true>{}, bool_c<true>{});
        else if (blo)
            chunk_loop(bool_c<false>{}, bool_c<true>{});
        else
            chunk_loop(bool_c<false>{}, bool_c<false>{});
    } else {
        chunk_loop(bool_c<true>{}, bool_c<true>{});
    }
    __builtin_amdgcn_s_setprio(0);
    if (tid == 0) next_tile = lo + taken;  // read after the end-of-tile barrier
    if (tid < kSrcTile) {
        const bool in = p0 + tid < HW;
        sm.org[tid][0] = in ? floor_clamped(sm.crd[0][tid]) : -(1 << 20);  // matches no cell
        sm.org[tid][1] = in ? floor_clamped(sm.crd[1][tid]) : -(1 << 20);
    }
    lds_barrier();  // every wave is done with the stages before T overwrites them

    // ---- window extraction ----
    // rows of level l inside this tile: [lr0[l], lr1[l]] (empty: lr0 > lr1)
    int lr0[kMaxLevels], lr1[kMaxLevels];
#pragma unroll
    for (int l = 0; l < kMaxLevels; l++) {
        lr0[l] = 1 << 30;
        lr1[l] = -(1 << 30);
        if (l < g.levels) {
            const int a = std::max(t0, g.off[l]) - g.off[l];
            const int b = std::min(t0 + kTgtTile, g.off[l] + g.h[l] * g.w[l]) - 1 - g.off[l];
            if (a <= b) {
                lr0[l] = a / g.w[l];
                lr1[l] = b / g.w[l];
            }
        }
    }
    // accumulator layout of the 32x32 MFMA: lane l, register v holds
    // D[i][j] with j = l % 32 (target) and i = 8*(v/4) + 4*(l/32) + v%4 (source)
    const int khalf = lane >> 5;
    // extraction: lane = (source g8 of a group of 8, window column cx). A wave
    // takes its 16 columns of T (sources) as two groups of 8 and walks the 8
    // window rows, so every read and store instruction covers 8 sources x 8
    // consecutive cells and all per-source set-up is plain per-lane arithmetic.
    const int g8 = lane >> 3, cx = lane & 7;
    // Window stores go through a buffer resource over this edge's window slot:
    // a lane whose cell is not stored (outside the tile, the grid or the
    // source range) gets an offset past the slot's size, and the hardware
    // discards the store. Every store instruction is then issued without a
    // branch around it.
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        win + win_index(slot0 + e, 0, 0, HW, 0), 0, kMaxLevels * 64 * HW * (int)sizeof(float),
        kBufWord3);

#pragma unroll
    for (int sb = 0; sb < 2; sb++) {
        if (sb) lds_barrier();  // the first half's cells have all been read
#pragma unroll
        for (int tb = 0; tb < 4; tb++)
#pragma unroll
            for (int gq = 0; gq < 4; gq++) {
                const int t = wn * 128 + tb * 32 + orow;
                const int s = wm * 32 + gq * 8 + khalf * 4;
                *reinterpret_cast<float4*>(&sm.u.T[t][s]) =
                    make_float4(acc[sb][tb][4 * gq], acc[sb][tb][4 * gq + 1],
                                acc[sb][tb][4 * gq + 2], acc[sb][tb][4 * gq + 3]);
            }
        lds_barrier();
#pragma unroll
        for (int grp = 0; grp < 2; grp++) {
            const int s = wave * 16 + grp * 8 + g8;                 // column of T
            const int lsrc = (s >> 5) * 64 + sb * 32 + (s & 31);   // source in the tile
            const int fx = sm.org[lsrc][0], fy = sm.org[lsrc][1];
            const bool pin = p0 + lsrc < HW;
            const float* Tcol = &sm.u.T[0][s];
            // byte offset of cell (cx, row 0) of level 0 in the slot
            const int woff = (int)win_index(0, 0, cx, HW, sm.pix[lsrc]) * 4;
#pragma unroll
            for (int l = 0; l < kMaxLevels; l++) {
                if (lr0[l] > lr1[l]) continue;  // level not in this tile
                const int wl = g.w[l], hl = g.h[l];
                const int ox = (fx >> l) - 3, oy = (fy >> l) - 3;
                const int xs = ox + cx;
                const bool colok = pin && (unsigned)xs < (unsigned)wl;
                // tile row of cell (cx, 0); wraps harmlessly for far origins
                // (then xs or the rows are out of range)
                unsigned tl = (unsigned)(g.off[l] - t0) + (unsigned)oy * (unsigned)wl +
                              (unsigned)xs;
                unsigned ta = tl * (unsigned)kTStride;  // offset of row tl in T
                float v[8];
                bool ok[8];  // this lane's cell of window row cy is in the tile and grid
#pragma unroll
                for (int cy = 0; cy < 8; cy++) {
                    ok[cy] = colok && (unsigned)(oy + cy) < (unsigned)hl &&
                             tl < (unsigned)kTgtTile;
                    v[cy] = Tcol[ok[cy] ? ta : 0u];
                    tl += (unsigned)wl;
                    ta += (unsigned)wl * (unsigned)kTStride;
                }
#pragma unroll
                for (int cy = 0; cy < 8; cy++)
                    __builtin_amdgcn_raw_buffer_store_b32(
                        __builtin_bit_cast(unsigned, fs * v[cy]), wrs,
                        ok[cy] ? woff + (l * 8 + cy) * HW * 32 : kBufDiscard, 0, 0);
            }
        }
    }
    lds_barrier();  // T is free again, next_tile is visible
    }
}

Geom make_geom(const slk_ctx* ctx) {
    Geom g{};
    g.HW = ctx->HW;
    g.C = ctx->C;
    g.levels = ctx->levels;
    int t = 0;
    for (int l = 0; l < kMaxLevels; l++) {
        g.h[l] = l < ctx->levels ? ctx->lh[l] : 0;
        g.w[l] = l < ctx->levels ? ctx->lw[l] : 1;
        g.off[l] = t;
        if (l < ctx->levels) {
            t += g.h[l] * g.w[l];
        }
    }
    g.Ttot = t;
    return g;
}

// u16 elements of one frame slot: the hi and lo planes [C/16][Ttot][16], then
// the frame's inverse split scale (one float), padded to 256 bytes
size_t slot_elems(const Geom& g) {
    return (2 * (size_t)g.C * g.Ttot + 2 + 127) / 128 * 128;
}

// the split of fp32 (or fp16) features under the context's precision
int split_mode(const slk_ctx* ctx) {
    return ctx->corr_prec == SLK_PREC_BF16X3 ? kSplitBF16 : kSplitF16;
}

// the preparation of nslots frame slots and, when mk.list is set, the tile
// mask of mk.nedges edges, in one launch
template <typename Tin>
int prep_slots_to(slk_ctx* ctx, const Tin* fm, long fstride, const SlotFrames& sf, const Geom& g,
                  int slot_lo, int nslots, bool pooled, const MaskArgs& mk, unsigned short* out,
                  int mode, hipStream_t stream) {
    const int nbx = (g.w[0] + kPrepCols - 1) / kPrepCols;
    const int nblk = nbx * ((g.h[0] + kPrepRows - 1) / kPrepRows);
    const long nprep = (long)nblk * (g.C / kChunk) * std::max(nslots, 0);
    const long nmask = mk.list ? mk.nedges : 0;
    if (nprep + nmask == 0) return SLK_OK;
    if (nprep + nmask > INT_MAX) return fail(SLK_E_ARG, "feature preparation grid too large");
    // vector loads of 4 pixels when every row starts 4-element aligned
    const bool vec = g.w[0] % 4 == 0 && fstride % 4 == 0 &&
                     reinterpret_cast<uintptr_t>(fm) % (4 * sizeof(Tin)) == 0;
    const long se = (long)slot_elems(g);
    float* part = ctx->frame_max.as<float>();
    const long n = (long)g.C * g.HW;
    const int nparts = (int)std::min<long>(kMaxParts, (n + kMaxChunk - 1) / kMaxChunk);
    if (mode == kSplitF16 && nslots > 0) {
        // the frames' partial maxima for their split scales
        if (ctx->frame_max.bytes < (size_t)(slot_lo + nslots) * kMaxParts * sizeof(float))
            return fail(SLK_E_ARG, "feature preparation: frame-maximum buffer too small");
        ProfScope ps(ctx, "corr_frame_max", stream);
        hipLaunchKernelGGL((k_frame_max<Tin>), dim3(nparts, nslots), dim3(256), 0, stream, fm,
                           fstride, sf, slot_lo, n, (vec && g.HW % 4 == 0) ? 1 : 0, nparts, part);
        SLK_HIP(hipGetLastError());
    }
    ProfScope ps(ctx, "corr_feat_prep", stream);
    // 1024-thread workgroups (16-wave mask chains) for maps up to 4096
    // pixels, two a CU; 512 above, three a CU (the preparation's share of
    // the launch is larger there)
    if (g.HW <= 4096)
        hipLaunchKernelGGL((k_feat_prep<Tin, 1024>), dim3((unsigned)(nprep + nmask)), dim3(1024),
                           0, stream, fm, fstride, sf, slot_lo, out, se, g, pooled ? 1 : 0,
                           vec ? 1 : 0, nbx, nblk, (int)nmask, mk, mode, part, nparts);
    else
        hipLaunchKernelGGL((k_feat_prep<Tin, 512>), dim3((unsigned)(nprep + nmask)), dim3(512),
                           0, stream, fm, fstride, sf, slot_lo, out, se, g, pooled ? 1 : 0,
                           vec ? 1 : 0, nbx, nblk, (int)nmask, mk, mode, part, nparts);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

template <typename Tin>
int prep_slots(slk_ctx* ctx, const Tin* fm, long fstride, const SlotFrames& sf, const Geom& g,
               int slot_lo, int nslots, bool pooled, const MaskArgs& mk, int mode,
               hipStream_t stream) {
    return prep_slots_to(ctx, fm, fstride, sf, g, slot_lo, nslots, pooled, mk,
                         ctx->split_feat.as<unsigned short>(), mode, stream);
}

// The tile-mask workgroups (with the preparation of nslots slots when
// nslots > 0) and the window kernel over `feat`, for edges whose slots are es.
// mode: the split of `feat`; alo: whether its level-0 lo planes can be
// nonzero (not for fp16 features under the fp16 split).
template <typename Tin>
int mask_and_windows(slk_ctx* ctx, const Tin* fm, long fstride, const SlotFrames& sf,
                     const Geom& g, int slot_lo, int nslots, bool pooled, const EdgeSlots& es,
                     const unsigned short* feat, int n, const float* coords, float* win,
                     int slot0, int mode, bool alo, hipStream_t stream) {
    const int mtiles = (g.HW + kSrcTile - 1) / kSrcTile;
    const int ntiles = (g.Ttot + kTgtTile - 1) / kTgtTile;
    const long total = (long)n * mtiles * ntiles;
    if (total > 0x7fffffffL) return fail(SLK_E_ARG, "correlation grid too large");
    if ((long)mtiles * ntiles > 32L * kPrepLdsWords)
        return fail(SLK_E_ARG, "correlation tiles per edge exceed the tile bitmap");
    MaskArgs mk{coords, ctx->tile_list.as<int>(), ctx->tile_ctr.as<int>(),
                ctx->src_order.as<int>(), mtiles, ntiles, n,
                ctx->mask_tab.as<unsigned long long>()};
    // feature preparation and the tile mask, one launch (after the frames'
    // maxima under the fp16 split)
    SLK_TRY(prep_slots(ctx, fm, fstride, sf, g, slot_lo, nslots, pooled, mk, mode, stream));
    {
        ProfScope ps(ctx, "corr_window", stream);
        const long se = (long)slot_elems(g);
        if (mode == kSplitF16)
            hipLaunchKernelGGL(k_corr_split_win<true>, dim3(ctx->ws_grid), dim3(256), 0, stream,
                               feat, se, es, ctx->src_order.as<int>(), win, slot0, g, ctx->alpha,
                               mtiles, ntiles, n, ctx->tile_list.as<int>(),
                               ctx->tile_ctr.as<int>(), alo ? 1 : 0);
        else
            hipLaunchKernelGGL(k_corr_split_win<false>, dim3(ctx->ws_grid), dim3(256), 0, stream,
                               feat, se, es, ctx->src_order.as<int>(), win, slot0, g, ctx->alpha,
                               mtiles, ntiles, n, ctx->tile_list.as<int>(),
                               ctx->tile_ctr.as<int>(), 1);
    }
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

template <typename Tin>
int split_windows(slk_ctx* ctx, const Tin* fm, long fstride, const int* ii_host,
                  const int* jj_host, const int* ii_dev, const int* jj_dev, int n,
                  const float* coords, float* win, int slot0, hipStream_t stream) {
    const Geom g = make_geom(ctx);
    SlotFrames sf{};
    EdgeSlots es{};
    const unsigned short* feat = ctx->split_feat.as<unsigned short>();
    const int mode = split_mode(ctx);
    const bool alo = !(mode == kSplitF16 && std::is_same<Tin, _Float16>::value);
    if (ii_host) {
        int ns = 0;
        auto slot_of = [&](int f) {
            for (int s = 0; s < ns; s++)
                if (sf.f[s] == f) return s;
            sf.f[ns] = f;
            return ns++;
        };
        for (int e = 0; e < n; e++) {
            es.si[e] = slot_of(ii_host[e]);
            es.sj[e] = slot_of(jj_host[e]);
        }
        return mask_and_windows(ctx, fm, fstride, sf, g, 0, ns, true, es, feat, n, coords, win,
                                slot0, mode, alo, stream);
    }
    sf.da = ii_dev;
    sf.db = jj_dev;
    sf.nb = n;
    for (int e = 0; e < n; e++) {
        es.si[e] = e;
        es.sj[e] = n + e;
    }
    // sources only need level 0 (their own launch); targets need every level
    {
        const MaskArgs none{nullptr, nullptr, nullptr, nullptr, 0, 0, 0, nullptr};
        SLK_TRY(prep_slots(ctx, fm, fstride, sf, g, 0, n, false, none, mode, stream));
    }
    return mask_and_windows(ctx, fm, fstride, sf, g, n, n, true, es, feat, n, coords, win, slot0,
                            mode, alo, stream);
}

}  // namespace

bool corr_split_supported(const slk_ctx* ctx) { return ctx->C % kChunk == 0; }

void corr_split_footprint(const slk_ctx* ctx, size_t* slot_bytes, size_t* tiles_per_edge,
                          size_t* order_per_edge, size_t* ctr_bytes, size_t* max_per_slot) {
    *max_per_slot = kMaxParts * sizeof(float);
    const Geom g = make_geom(ctx);
    const size_t mtiles = (g.HW + kSrcTile - 1) / kSrcTile;
    const size_t ntiles = (g.Ttot + kTgtTile - 1) / kTgtTile;
    *slot_bytes = slot_elems(g) * sizeof(unsigned short);
    *tiles_per_edge = mtiles * ntiles * sizeof(int);
    *order_per_edge = 3 * (size_t)g.HW * sizeof(int);
    *ctr_bytes = kCtrInts * sizeof(int);
}

int corr_split_grid(int cus) { return std::max(8, cus / 8 * 8) * 2; }

int corr_split_alloc(slk_ctx* ctx) {
    if (!corr_split_supported(ctx)) return SLK_OK;
    const Geom g = make_geom(ctx);
    const size_t slots = 2 * (size_t)std::min(ctx->max_batch, kMaxEdgesPerLaunch);
    SLK_TRY(ctx->split_feat.ensure(slots * slot_elems(g) * sizeof(unsigned short)));
    SLK_TRY(ctx->frame_max.ensure(slots * kMaxParts * sizeof(float)));
    const size_t mtiles = (g.HW + kSrcTile - 1) / kSrcTile;
    const size_t ntiles = (g.Ttot + kTgtTile - 1) / kTgtTile;
    const size_t tiles = (size_t)std::min(ctx->max_batch, kMaxEdgesPerLaunch) * mtiles * ntiles;
    SLK_TRY(ctx->tile_list.ensure(tiles * sizeof(int)));
    SLK_TRY(ctx->src_order.ensure((size_t)std::min(ctx->max_batch, kMaxEdgesPerLaunch) * 3 *
                                  g.HW * sizeof(int)));
    SLK_TRY(ctx->tile_ctr.ensure(kCtrInts * sizeof(int)));
    if (ntiles <= 64) {  // tile masks as 64-bit words: their table by position
        const long entries = (long)(g.w[0] + 2 * kTabPad) * (g.h[0] + 2 * kTabPad);
        SLK_TRY(ctx->mask_tab.ensure((size_t)entries * sizeof(unsigned long long)));
        hipLaunchKernelGGL(k_mask_table, dim3((unsigned)((entries + 255) / 256)), dim3(256), 0, 0,
                           g, ctx->mask_tab.as<unsigned long long>());
        SLK_HIP(hipGetLastError());
    }
    // the correlation workgroups: two per CU, a multiple of the 8 XCDs
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, ctx->device) !=
        hipSuccess)
        return fail(SLK_E_HIP, "hipDeviceGetAttribute(multiProcessorCount) failed");
    ctx->ws_grid = corr_split_grid(cus);
    return SLK_OK;
}

int corr_split_windows(slk_ctx* ctx, const void* fmaps, int dtype, long fstride,
                       const int* ii_host, const int* jj_host, const int* ii_dev,
                       const int* jj_dev, int n, const float* coords, float* win, int slot0,
                       hipStream_t stream) {
    if (n <= 0) return SLK_OK;
    if (n > kMaxEdgesPerLaunch || n > ctx->max_batch)
        return fail(SLK_E_ARG, "corr_split_windows: too many edges for one launch");
    if (dtype == SLK_F32)
        return split_windows(ctx, static_cast<const float*>(fmaps), fstride, ii_host, jj_host,
                             ii_dev, jj_dev, n, coords, win, slot0, stream);
    return split_windows(ctx, static_cast<const _Float16*>(fmaps), fstride, ii_host, jj_host,
                         ii_dev, jj_dev, n, coords, win, slot0, stream);
}


int corr_split_prepare(slk_ctx* ctx, const void* fmaps, int dtype, long fstride, int nframes,
                       hipStream_t stream) {
    if (nframes <= 0) return fail(SLK_E_ARG, "corr_prepare_frames: nframes <= 0");
    const Geom g = make_geom(ctx);
    const size_t bytes = (size_t)nframes * slot_elems(g) * sizeof(unsigned short);
    if (bytes > ctx->prep_feat.bytes && ctx->prep_feat.ptr)
        SLK_HIP(hipDeviceSynchronize());  // earlier launches may still read the old frames
    SLK_TRY(ctx->prep_feat.ensure(bytes));
    if ((size_t)nframes * kMaxParts * sizeof(float) > ctx->frame_max.bytes && ctx->frame_max.ptr)
        SLK_HIP(hipDeviceSynchronize());  // earlier launches may still read the old maxima
    SLK_TRY(ctx->frame_max.ensure((size_t)nframes * kMaxParts * sizeof(float)));
    SlotFrames sf{};
    sf.ident = 1;
    const MaskArgs none{nullptr, nullptr, nullptr, nullptr, 0, 0, 0, nullptr};
    const int mode = split_mode(ctx);
    if (dtype == SLK_F32)
        SLK_TRY(prep_slots_to(ctx, static_cast<const float*>(fmaps), fstride, sf, g, 0, nframes,
                              true, none, ctx->prep_feat.as<unsigned short>(), mode, stream));
    else
        SLK_TRY(prep_slots_to(ctx, static_cast<const _Float16*>(fmaps), fstride, sf, g, 0,
                              nframes, true, none, ctx->prep_feat.as<unsigned short>(), mode,
                              stream));
    ctx->prep_nframes = nframes;
    ctx->prep_mode = mode;
    ctx->prep_alo = !(mode == kSplitF16 && dtype == SLK_F16);
    return SLK_OK;
}

int corr_split_windows_prepared(slk_ctx* ctx, const int* ii_host, const int* jj_host, int n,
                                const float* coords, float* win, int slot0, hipStream_t stream) {
    if (n <= 0) return SLK_OK;
    if (n > kMaxEdgesPerLaunch || n > ctx->max_batch)
        return fail(SLK_E_ARG, "corr_split_windows: too many edges for one launch");
    const Geom g = make_geom(ctx);
    EdgeSlots es{};
    for (int e = 0; e < n; e++) {
        es.si[e] = ii_host[e];
        es.sj[e] = jj_host[e];
    }
    const SlotFrames none{};
    return mask_and_windows(ctx, static_cast<const float*>(nullptr), 0, none, g, 0, 0, true, es,
                            ctx->prep_feat.as<unsigned short>(), n, coords, win, slot0,
                            ctx->prep_mode, ctx->prep_alo, stream);
}

}  // namespace slk
