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
// Stage 1 (k_feat_prep), once per frame a launch uses: the fp32 pooled
// features of levels 1..3 (formed in LDS from level 0) and a hi/lo split of
// every pixel of all levels, stored chunk-major [plane][C/16][rows][16] so a
// 16-channel chunk of consecutive rows is one contiguous block, followed by
// one float per row: the inverse of the row's split scale.
//   fp16 split (SLK_PREC_F16X3, the default): a pixel's features are scaled
//   by one power of two 2^e chosen from their largest magnitude m over the
//   channels (m * 2^e in [2^14, 2^15)), then hi = rne_f16(x 2^e),
//   lo = rne_f16(x 2^e - hi): 22 significant bits relative to m, the
//   dropped lo.lo term ~2^-22 m_i m_j per product of pixels i and j. fp16
//   features are taken with e >= 0, which makes hi exact and lo zero at
//   level 0.
//   bf16 split (SLK_PREC_BF16X3): hi = rne_bf16(x), lo = rne_bf16(x - hi),
//   no scale (16 significant bits, lo.lo ~2^-16).
// Stage 2 (order_and_boxes, workgroups of the same launch as stage 1): each
// edge's sources sorted by where their windows fall, runs of 128 of them
// (source tiles) with the bounding box of their windows at every level; the
// boxes' cells are a source tile's "virtual" targets, listed in tiles of 256.
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
// sources' windows, multiplied by alpha times both pixels' inverse scales
// (powers of two: the scaling adds no rounding). Only ~2% of the level-0 products are
// window cells, and none of them costs more than its LDS round trip.
#include <algorithm>
#include <climits>
#include <type_traits>

#include "corr_common.hpp"
#include "lds_dma.hpp"

namespace slk {
namespace {

constexpr int kSrcTile = 128;  // sources per workgroup
constexpr int kTgtTile = 256;  // targets per workgroup
constexpr int kChunk = 16;     // channels per LDS stage
constexpr int kStages = 3;     // LDS stages: chunk k+2 streams in while chunk k is used
constexpr int kTStride = 68;   // floats per transposed-tile row (64 sources + 4 pad)
constexpr int kTPad = 3;       // rows of the transposed tile before and after its targets
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

// Source order and target boxes of an edge (one workgroup per edge, in the
// launch of k_feat_prep beside the feature preparation it does not depend on).
//
// Sources are ordered by where their windows fall: the floored coordinates
// (fx, fy), clamped to [-8, w] x [-8, h] (a window of a source outside that
// range meets the level-0 image nowhere, and the clamp keeps it beside the
// sources whose pooled-level windows it shares), fall in bands of kBand rows;
// the bands are walked top to bottom and within a band the columns snake
// (left to right in even bands, right to left in odd ones), so that a run of
// 128 sorted sources -- a source tile -- covers about a 16 x 8 pixel patch of
// the target frame, and a run crossing into the next band stays at the same
// image side. Columns are taken in groups of 2^sx when the map is too wide for
// kMaxKeys buckets.
//
// A source tile's target box at level l is the bounding box of its sources'
// 8x8 windows there, clipped to the level: from the bucket range of its
// first and last sorted source, every source of the tile lies in that range
// of bands and column groups, and the box of the range's floored extremes
// holds all of their in-grid window cells. The tile's target rows are the
// boxes' cells concatenated (level 0 first, each box row-major), a "virtual"
// target list cut into runs of kTgtTile: k_corr_split_win gathers its target
// tile's operand rows through the box arithmetic, so a source tile computes
// its own windows' neighbourhood only. Which tile computes a window cell
// changes no result: a cell is the same dot product of the same operand rows.
//
// Per edge: a counting sort over the keys (LDS histogram by atomic adds, an
// exclusive scan, a scatter by atomic slot claims: the order within a bucket
// is not fixed, the bucket ranges are), ord[q] = pixel at sorted position q
// (claimed in LDS and written out in order when the keys leave room); the
// boxes of each source tile as kBoxInts ints (ya, xa, bh, bw per level)
// after them; the (source tile,
// virtual tile) ids mt * ntiles + vt into the edge's segment list[e * tpe ..]
// and their number into ctr[kCtrCount + e]. Edge 0 also zeroes the tile
// counters of k_corr_split_win, which runs after this on the same stream.
// LDS of an order workgroup (arrays of the preparation's, reused): the
// bucket counts of the sort, and the virtual tile counts of the source tiles
constexpr int kPrepLdsWords = 8192;
constexpr int kPrepL1Words = 2048;
constexpr int kBand = 16;                 // image rows per band of the source order
constexpr int kMaxKeys = kPrepLdsWords;   // buckets of the sort
constexpr int kBoxInts = 4 * kMaxLevels;  // per source tile: ya, xa, bh, bw of each level
constexpr int kCtrXcd = 0;     // [0..7] next list index of each XCD's eighth
constexpr int kCtrCount = 8;   // [8..8+edges) listed tiles of each edge
constexpr int kCtrInts = kCtrCount + kMaxEdgesPerLaunch;

// the bucket layout of the sort: nxb column groups of 2^sx columns, nkeys
// buckets in all
struct KeyGeom {
    int nxb, sx, nkeys;
};

KeyGeom key_geom(const Geom& g) {
    const int kx = g.w[0] + 9, nb = (g.h[0] + 9 + kBand - 1) / kBand;
    KeyGeom k{kx, 0, nb * kx};
    while (k.nkeys > kMaxKeys && k.sx < 20) {
        k.sx++;
        k.nxb = (kx + (1 << k.sx) - 1) >> k.sx;
        k.nkeys = nb * k.nxb;
    }
    return k;
}

struct MaskArgs {
    const float* coords;
    int* list;
    int* ctr;
    int* order;   // [edge][ostride]: pixel of each sorted position, then the boxes
    long ostride;
    int mtiles, ntiles, nedges;
    KeyGeom kg;
};

// ints of an edge's order record: HW pixels, then kBoxInts per source tile
__host__ __device__ __forceinline__ long order_stride(int HW, int mtiles) {
    return (long)HW + (long)kBoxInts * mtiles;
}

__device__ __forceinline__ int sort_key(const KeyGeom& k, const Geom& g, int fx, int fy) {
    const int band = (std::min(std::max(fy, -8), g.h[0]) + 8) / kBand;
    const int xb = (std::min(std::max(fx, -8), g.w[0]) + 8) >> k.sx;
    return band * k.nxb + ((band & 1) ? k.nxb - 1 - xb : xb);
}

// The boxes of a source tile whose sorted sources fall in buckets b0..b1
// (b0 <= b1), as (ya, xa, bh, bw) of each level (an empty level has bh = bw = 0).
__device__ __forceinline__ void tile_boxes(const KeyGeom& k, const Geom& g, int b0, int b1,
                                           int* rec) {
    const int n = k.nxb;
    const int band0 = b0 / n, band1 = b1 / n;
    auto col = [&](int b) {  // column group of bucket b
        const int s = b % n;
        return ((b / n) & 1) ? n - 1 - s : s;
    };
    const int c0 = col(b0), c1 = col(b1);
    int xlo = 0, xhi = n - 1;  // bands b0 .. b1 two or more apart: every column
    if (band0 == band1) {
        xlo = std::min(c0, c1);
        xhi = std::max(c0, c1);
    } else if (band1 == band0 + 1) {  // both partial bands end at the same side
        if (band0 & 1)
            xhi = std::max(c0, c1);
        else
            xlo = std::min(c0, c1);
    }
    // floored coordinate range (of the clamped coordinates: a source clamped
    // at a side has its in-grid cells inside the box of the clamp value)
    const int fx0 = (xlo << k.sx) - 8, fx1 = ((xhi + 1) << k.sx) - 9;
    const int fy0 = band0 * kBand - 8, fy1 = band1 * kBand + kBand - 9;
#pragma unroll
    for (int l = 0; l < kMaxLevels; l++) {
        const int xa = std::max((fx0 >> l) - 3, 0), xb = std::min((fx1 >> l) + 4, g.w[l] - 1);
        const int ya = std::max((fy0 >> l) - 3, 0), yb = std::min((fy1 >> l) + 4, g.h[l] - 1);
        const bool in = l < g.levels && xa <= xb && ya <= yb;
        rec[4 * l] = in ? ya : 0;
        rec[4 * l + 1] = in ? xa : 0;
        rec[4 * l + 2] = in ? yb - ya + 1 : 0;
        rec[4 * l + 3] = in ? xb - xa + 1 : 0;
    }
}

// Exclusive prefix sums of a[0..n) in place (LDS), by all kT threads; returns
// the total. Each thread takes a contiguous run, the runs' sums are scanned
// in the waves and across them through wsum (kT / 64 ints).
template <int kT>
__device__ int scan_excl(int* a, int n, int* wsum) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int per = (n + kT - 1) / kT;
    const int i0 = std::min(n, tid * per), i1 = std::min(n, i0 + per);
    int s = 0;
    for (int i = i0; i < i1; i++) s += a[i];
    int incl = s;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int v = __shfl_up(incl, off, 64);
        if (lane >= off) incl += v;
    }
    if (lane == 63) wsum[wv] = incl;
    __syncthreads();
    int before = incl - s, total = 0;
#pragma unroll
    for (int w = 0; w < kT / 64; w++) {
        const int v = wsum[w];
        before += w < wv ? v : 0;
        total += v;
    }
    for (int i = i0; i < i1; i++) {
        const int c = a[i];
        a[i] = before;
        before += c;
    }
    __syncthreads();  // a is complete; wsum may be reused
    return total;
}

// keys: kPrepLdsWords ints of LDS (the bucket counts, then the sorted pixels
// when they fit), ntv: mtiles ints of LDS
template <int kT>
__device__ void order_and_boxes(const MaskArgs& a, const Geom& g, int e, int* keys, int* ntv,
                                int* wsum) {
    const int tid = threadIdx.x;
    const int HW = g.HW, mtiles = a.mtiles, ntiles = a.ntiles;
    const KeyGeom kg = a.kg;
    const float* cc = a.coords + (size_t)e * 2 * HW;
    int* ord = a.order + (size_t)e * a.ostride;
    int* rec = ord + HW;
    // the sorted pixels are claimed in LDS and stored in order afterwards
    // (scattered 4-byte stores from one workgroup are slow); a map too large
    // for that scatters them to ord directly
    int* spix = kg.nkeys + HW <= kPrepLdsWords ? keys + kg.nkeys : nullptr;
    for (int i = tid; i < kg.nkeys; i += kT) keys[i] = 0;
    if (e == 0 && tid < 8) a.ctr[kCtrXcd + tid] = 0;
    __syncthreads();
    // A thread's sources are p = tid + u * kT; up to kU of them stay in
    // registers between the counting and the scatter (a map of more than
    // kU * kT pixels loads its coordinates again for the scatter).
    constexpr int kU = kT >= 1024 ? 4 : 12;
    const bool keep = HW <= kU * kT;
    int kv[kU];
    float xv[kU], yv[kU];
    auto load = [&](int p0) {
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const int p = std::min(p0 + u * kT + tid, HW - 1);
            xv[u] = cc[p];
            yv[u] = cc[HW + p];
        }
#pragma unroll
        for (int u = 0; u < kU; u++)
            kv[u] = sort_key(kg, g, floor_clamped(xv[u]), floor_clamped(yv[u]));
    };
    for (int p0 = 0; p0 < HW; p0 += kU * kT) {
        load(p0);
#pragma unroll
        for (int u = 0; u < kU; u++)
            if (p0 + u * kT + tid < HW) atomicAdd(&keys[kv[u]], 1);
    }
    __syncthreads();
    scan_excl<kT>(keys, kg.nkeys, wsum);  // keys[b]: first sorted position of bucket b
    for (int p0 = 0; p0 < HW; p0 += kU * kT) {
        if (!keep) load(p0);
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const int p = p0 + u * kT + tid;
            if (p < HW) {
                const int q = atomicAdd(&keys[kv[u]], 1);
                if (spix)
                    spix[q] = p;
                else
                    ord[q] = p;
            }
        }
    }
    __syncthreads();  // keys[b]: one past the last sorted position of bucket b
    if (spix)
        for (int i = tid; i < HW; i += kT) ord[i] = spix[i];
    // bucket of sorted position q: the first b whose end exceeds q
    auto bucket_of = [&](int q) {
        int lo = 0, hi = kg.nkeys - 1;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (keys[mid] > q)
                hi = mid;
            else
                lo = mid + 1;
        }
        return lo;
    };
    for (int mt = tid; mt < mtiles; mt += kT) {
        int r[kBoxInts];
        tile_boxes(kg, g, bucket_of(mt * kSrcTile), bucket_of(std::min(mt * kSrcTile + kSrcTile, HW) - 1),
                   r);
        int total = 0;
#pragma unroll
        for (int i = 0; i < kBoxInts; i++) rec[(size_t)mt * kBoxInts + i] = r[i];
#pragma unroll
        for (int l = 0; l < kMaxLevels; l++) total += r[4 * l + 2] * r[4 * l + 3];
        ntv[mt] = (total + kTgtTile - 1) / kTgtTile;
    }
    __syncthreads();
    const int count = scan_excl<kT>(ntv, mtiles, wsum);  // ntv[mt]: first list slot of mt
    int* seg = a.list + (size_t)e * mtiles * ntiles;
    for (int mt = tid; mt < mtiles; mt += kT) {
        const int s0 = ntv[mt], s1 = mt + 1 < mtiles ? ntv[mt + 1] : count;
        for (int s = s0; s < s1; s++) seg[s] = mt * ntiles + (s - s0);
    }
    if (tid == 0) a.ctr[kCtrCount + e] = count;
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

// The exponent e of a pixel's fp16 split scale 2^e from its largest magnitude
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

// Feature preparation of frame slots, one launch of 1024-thread workgroups.
// A workgroup takes an 8 x 32 block of level-0 pixels; wave w holds block
// rows 2 (w % 4) (lanes 0-31) and 2 (w % 4) + 1 (lanes 32-63) of channel
// group w / 4 (32 channels of a pixel in a thread's registers), so each load
// instruction reads two 128-byte row pieces. A pixel's split scale comes
// from the largest magnitude among its channels (the four groups' maxima
// through LDS); its thread writes the hi/lo split of its two chunks, 16
// channels = 32 bytes per pixel and plane, into
// out[slot][plane][C/16][Ttot][16], and group 0 the pixel's inverse scale
// into the slot's float array [Ttot] after the planes. Pooled levels (each
// pooled value 0.25 * (((a + b) + c) + d) of its 2x2 parents, the parents'
// row first; a pooled pixel's parents always lie in the block): level 1 in
// registers (the 2x2 parents of level-1 pixel (w % 4, x) are lanes 2x,
// 2x + 1, 2x + 32, 2x + 33 of the wave: quad moves and a cross-half
// permute), kept by lane 2x; level 2 from level 1 through LDS, level 3
// from level 2 by quad moves; a level-2 or level-3 pixel's channels of a
// group are collected by one owner thread (lanes 32.. of the group's waves).
// Under the fp16 split a pixel's features are scaled by 2^e (split_exponent
// of its largest magnitude), under the bf16 split by 1. `pooled` = 0 writes
// level 0 only (source slots).
// One-dimensional grid: first, when mk.list is set, one order workgroup per
// edge (order_and_boxes, on the exchange arrays; they are the longer chains,
// so they are dispatched first), then the blocks x slots preparation
// workgroups, renumbered so that each XCD (workgroups are dealt to the 8 XCDs
// in turn) takes a contiguous run of blocks.
constexpr int kPrepC = 128;          // channels of the split path, at most
constexpr int kPW = 32, kPH = 8;     // block columns and rows
constexpr int kPGrp = 4;             // channel groups
constexpr int kPGc = kPrepC / kPGrp; // channels of a group (two chunks)
constexpr int kPN1 = (kPH / 2) * (kPW / 2), kPN2 = (kPH / 4) * (kPW / 4), kPN3 = kPW / 8;
static_assert(kPGrp * kPH * kPW == 1024 && kPGc == 2 * kChunk, "prep workgroup shape");

__device__ __forceinline__ float pool4(float a, float b, float c, float d) {
    return 0.25f * (((a + b) + c) + d);
}

// v of another lane of the caller's quad (DPP quad_perm kCtrl)
template <int kCtrl>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), kCtrl,
                                                              0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xB1;                                       // quad_perm(1, 0, 3, 2)
constexpr int kDppQ1 = 0x55, kDppQ2 = 0xAA, kDppQ3 = 0xFF;           // quad_perm(k, k, k, k)

// the hi/lo split of one pixel's chunk k (16 channels) at row t
__device__ __forceinline__ void emit_chunk(unsigned short* slot, size_t plane, int Ttot, int k,
                                           int t, const float* v, float sc, int mode) {
    u16x8_t hi[2], lo[2];
#pragma unroll
    for (int u = 0; u < kChunk; u++) {
        const unsigned pk = mode == kSplitF16 ? split_f16(v[u] * sc) : split_bf16(v[u]);
        hi[u >> 3][u & 7] = (unsigned short)(pk & 0xffffu);
        lo[u >> 3][u & 7] = (unsigned short)(pk >> 16);
    }
    unsigned short* o = slot + ((size_t)k * Ttot + t) * kChunk;
    *reinterpret_cast<u16x8_t*>(o) = hi[0];
    *reinterpret_cast<u16x8_t*>(o + 8) = hi[1];
    *reinterpret_cast<u16x8_t*>(o + plane) = lo[0];
    *reinterpret_cast<u16x8_t*>(o + plane + 8) = lo[1];
}

template <typename Tin>
__global__ __launch_bounds__(1024) void k_feat_prep(
    const Tin* __restrict__ fm, long fstride, SlotFrames sf, int slot_lo,
    unsigned short* __restrict__ out, long slot_elems, Geom g, int pooled, int nbx, int nblk,
    int nmask, MaskArgs mk, int mode) {
    constexpr int kPN23 = kPN2 + kPN3;
    __shared__ float pl1[kPGrp][kPGc][kPH / 2][kPW / 2];  // level 1 of every group
    __shared__ float pl2[kPGrp][kPGc][kPN23];             // levels 2 and 3, row-major
    __shared__ float pmax[kPGrp][kPH * kPW];              // per group: max |x| of a pixel
    __shared__ float pmax1[kPGrp][kPN1];                  // ... of a level-1 pixel
    __shared__ float pmax23[kPGrp][kPN23];                // ... of a level-2 or 3 pixel
    __shared__ int wave_sum[16];
    if ((int)blockIdx.x < nmask) {  // uniform
        // the order chains are the launch's long pole: their waves issue
        // ahead of the preparation waves sharing their SIMDs
        __builtin_amdgcn_s_setprio(2);
        static_assert(sizeof(pl1) >= kMaxKeys * sizeof(int) &&
                          sizeof(pl2) >= kPrepL1Words * sizeof(int), "order LDS");
        order_and_boxes<1024>(mk, g, blockIdx.x, reinterpret_cast<int*>(&pl1[0][0][0][0]),
                              reinterpret_cast<int*>(&pl2[0][0][0]), wave_sum);
        return;
    }
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int q = wave >> 2, wr = wave & 3, gi = tid & 255;  // group, row pair, thread in group
    const int hf = lane >> 5, x = lane & 31, r = 2 * wr + hf;  // gi = r * kPW + x
    const int nprep = (int)gridDim.x - nmask;
    int b = blockIdx.x - nmask;
    {
        const int qq = nprep / 8;  // XCD b % 8 takes blocks (b % 8) qq .. + qq - 1
        if (b < 8 * qq) b = (b & 7) * qq + (b >> 3);
    }
    const int blk = b % nblk, s = slot_lo + b / nblk;
    const int bx = blk % nbx, by = blk / nbx;
    const int W = g.w[0], H = g.h[0], C = g.C, nk = C / kChunk;
    const int yy = by * kPH + r, xx = bx * kPW + x;
    const bool inmap = yy < H && xx < W;
    const Tin* src = fm + (long)slot_frame(sf, s) * fstride + (inmap ? (long)yy * W + xx : 0L);
    // the pixel's channels of group q (zero past C and outside the map): every
    // load unconditional (from a clamped, in-range address) and issued before
    // the first is used
    float v[kPGc];
#pragma unroll
    for (int i = 0; i < kPGc; i++) v[i] = ldf(src + (long)std::min(q * kPGc + i, C - 1) * g.HW);
    __builtin_amdgcn_sched_barrier(0);  // every load out before the first use
#pragma unroll
    for (int i = 0; i < kPGc; i++) v[i] = inmap && q * kPGc + i < C ? v[i] : 0.0f;
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < kPGc; i++) m = fmaxf(m, fabsf(v[i]));
    pmax[q][gi] = m;
    const bool pool = pooled && g.levels > 1;  // uniform
    // level-1 owners: lane 2 x1 of the lower half (pixel (wr, x1)); level-2
    // and level-3 owners: lanes 32.. of the group's waves, o23 = wr * 32 + x
    const bool own1 = hf == 0 && !(x & 1);
    const int o23 = wr * 32 + x;
    const bool own23 = hf == 1 && o23 < kPN23;
    float p[kPGc];
    if (pool) {
#pragma unroll
        for (int i = 0; i < kPGc; i++) {
            const float bq = dpp_f<kDppXor1>(v[i]);
            // lane xor 32 (ds_bpermute; this compiler's permlane32_swap
            // builtin returned the operand's own half here)
            const float cq = __builtin_bit_cast(
                float, __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, __builtin_bit_cast(int, v[i])));
            const float dq = dpp_f<kDppXor1>(cq);
            p[i] = pool4(v[i], bq, cq, dq);
        }
        float m1 = 0.0f;
#pragma unroll
        for (int i = 0; i < kPGc; i++) m1 = fmaxf(m1, fabsf(p[i]));
        if (own1) {
#pragma unroll
            for (int i = 0; i < kPGc; i++) pl1[q][i][wr][x >> 1] = p[i];
            pmax1[q][wr * (kPW / 2) + (x >> 1)] = m1;
        }
        lds_barrier();
        // level 2: (group, channel, x3, y2, x2 & 1) items, 2 a thread; the four
        // level-2 parents of a level-3 pixel are the lanes of a quad, whose
        // first lane pools them
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int i = tid + 1024 * u;
            const int gq = i >> 9, c = (i >> 4) & 31, x3 = (i >> 2) & 3;
            const int y2 = (i >> 1) & 1, x2 = 2 * x3 + (i & 1);
            const float l2 = pool4(pl1[gq][c][2 * y2][2 * x2], pl1[gq][c][2 * y2][2 * x2 + 1],
                                   pl1[gq][c][2 * y2 + 1][2 * x2], pl1[gq][c][2 * y2 + 1][2 * x2 + 1]);
            pl2[gq][c][y2 * (kPW / 4) + x2] = l2;
            const float l3 = pool4(l2, dpp_f<kDppQ1>(l2), dpp_f<kDppQ2>(l2), dpp_f<kDppQ3>(l2));
            if ((i & 3) == 0) pl2[gq][c][kPN2 + x3] = l3;
        }
        lds_barrier();
        if (own23) {
            float m23 = 0.0f;
#pragma unroll
            for (int i = 0; i < kPGc; i++) {
                p[i] = pl2[q][i][o23];
                m23 = fmaxf(m23, fabsf(p[i]));
            }
            pmax23[q][o23] = m23;
        }
    }
    lds_barrier();
    auto scale_of = [&](float pm) {
        return mode == kSplitF16 ? __builtin_amdgcn_ldexpf(
                                       1.0f, split_exponent(pm, std::is_same<Tin, _Float16>::value))
                                 : 1.0f;
    };
    const size_t plane = (size_t)C * g.Ttot;
    unsigned short* const slot = out + (size_t)s * slot_elems;
    float* const inv = reinterpret_cast<float*>(slot + 2 * plane);
    // every store after the LDS work: level 0, then the owned pooled pixel
    {
        float pm = 0.0f;
#pragma unroll
        for (int gq = 0; gq < kPGrp; gq++) pm = fmaxf(pm, pmax[gq][gi]);
        const float sc = scale_of(pm);
        if (inmap) {
            const int t = yy * W + xx;
#pragma unroll
            for (int j = 0; j < 2; j++)
                if (2 * q + j < nk)
                    emit_chunk(slot, plane, g.Ttot, 2 * q + j, t, &v[kChunk * j], sc, mode);
            if (q == 0) inv[t] = 1.0f / sc;  // a power of two: exact
        }
    }
    if (!pool || !(own1 || own23)) return;
    const int ol = own1 ? 1 : o23 < kPN2 ? 2 : 3;
    if (ol >= g.levels) return;
    const int oy = ol == 1 ? wr : ol == 2 ? o23 / (kPW / 4) : 0;
    const int ox = ol == 1 ? x >> 1 : ol == 2 ? o23 % (kPW / 4) : o23 - kPN2;
    const int ly = by * (kPH >> ol) + oy, lx = bx * (kPW >> ol) + ox;
    if (ly >= g.h[ol] || lx >= g.w[ol]) return;
    float pm = 0.0f;
#pragma unroll
    for (int gq = 0; gq < kPGrp; gq++)
        pm = fmaxf(pm, ol == 1 ? pmax1[gq][wr * (kPW / 2) + ox] : pmax23[gq][o23]);
    const float sc = scale_of(pm);
    const int t = g.off[ol] + ly * g.w[ol] + lx;
#pragma unroll
    for (int j = 0; j < 2; j++)
        if (2 * q + j < nk) emit_chunk(slot, plane, g.Ttot, 2 * q + j, t, &p[kChunk * j], sc, mode);
    if (q == 0) inv[t] = 1.0f / sc;
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
        // [kTPad + target][source] of one 64-source half; the kTPad rows on
        // either side are never written and only read for cells outside the
        // grid, which the lookup never reads
        float T[kTgtTile + 2 * kTPad][kTStride];
    } u;
    int org[kSrcTile][2];     // floor_clamped(x), floor_clamped(y) of each source
    float crd[2][kSrcTile];   // x, y coordinates of the tile's sources
    int pix[kSrcTile];        // pixel of each source
    float ssc[kSrcTile];      // alpha times each source's inverse split scale
    float tsc[kTgtTile];      // each target's inverse split scale
    // the next tile's list entry, box record and order pixels (pf_pix[i] =
    // ord[min(p0 + i, HW - 1)]), put here by direct-to-LDS loads while the
    // current tile's chunks stream
    int pf_r;
    int pf_rec[kBoxInts];
    int pf_pix[kSrcTile];
};

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
// listed tiles (order_and_boxes) one at a time from its XCD's counter: tile
// index idx runs over the edges' segments concatenated, workgroup blockIdx % 8
// runs on that XCD and serves the XCD's contiguous eighth of those indices,
// so the edges an XCD works on stay in its L2, and no CU idles while tiles
// remain. Waves form a 2x2 grid: wave (wm, wn) owns sources
// wm*64..+63 and targets wn*128..+127 of a tile, eight 32x32 accumulator
// blocks. Source tile mt holds sorted positions mt*128..+127 of the edge's
// order: the A rows and the coordinates are gathered through the order's
// pixels, the B rows through the tile's target boxes (virtual tile vt holds
// virtual rows vt*256..+255), and each source's windows are stored at its
// own pixel. kF16: fp16 operands (the scaled fp16
// split), else bf16. alo = 0: every source lo is zero (fp16 features, fp16
// split), and so is every level-0 target lo: a tile of level-0 targets then
// takes the one pass hi.hi, a tile with pooled targets hi.hi + hi.lo.
template <bool kF16>
__global__ __launch_bounds__(256, 2) void k_corr_split_win(
    const unsigned short* __restrict__ feat, long slot_elems, EdgeSlots es,
    const int* __restrict__ order, long ostride, const float* __restrict__ coords,
    float* __restrict__ win, int slot0, Geom g,
    float alpha, int mtiles, int ntiles, int nedges, const int* __restrict__ list,
    int* __restrict__ ctr, int alo) {
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
    // LDS after the chunk loop's first wait (which covers the atomic's return).
    int* const counter = ctr + kCtrXcd + xcd;
    // the edge of tile idx: the last lane whose prefix is <= idx (edges
    // with no marked tile share their successor's prefix)
    auto edge_of = [&](int idx) {
        const bool before_idx = (int)(threadIdx.x & 63) < nedges && pre <= idx;
        return (int)__builtin_popcountll(__ballot(before_idx)) - 1;
    };
    // A tile's metadata into sm.pf_*, in two dependent steps: its list entry
    // (thread 0), then its box record (lanes 0..15 of wave 0) and the order
    // pixels of its sources (waves 0 and 1). Each step's data is in LDS after
    // a vmcnt wait of the issuing waves and a barrier.
    auto pf_list = [&](int idx) {
        const int e = edge_of(idx);
        if (threadIdx.x == 0)
            dma_x1(list + (size_t)e * tpe + (idx - __builtin_amdgcn_readlane(pre, e)),
                   lds_addr(&sm.pf_r));
    };
    auto pf_rest = [&](int idx) {
        const int e = edge_of(idx);
        const int mt = __builtin_amdgcn_readfirstlane(sm.pf_r) / ntiles;
        const int* ord = order + (size_t)e * ostride;
        const int t = threadIdx.x;
        if (t < kBoxInts) dma_x1(ord + g.HW + mt * kBoxInts + t, lds_addr(&sm.pf_rec[0]));
        if (t < kSrcTile)
            dma_x1(ord + std::min(mt * kSrcTile + t, g.HW - 1), lds_addr(&sm.pf_pix[t & ~63]));
    };
    auto pf_sync = [&](int idx) {  // both steps, waiting for each
        pf_list(idx);
        __builtin_amdgcn_s_waitcnt(kWaitVm0Lgkm0);
        lds_barrier();
        pf_rest(idx);
        __builtin_amdgcn_s_waitcnt(kWaitVm0Lgkm0);
        lds_barrier();
    };
    if (threadIdx.x == 0) next_tile = lo + atomicAdd(counter, 1);
    lds_barrier();
    {
        const int idx0 = __builtin_amdgcn_readfirstlane(next_tile);
        if (idx0 < hi) pf_sync(idx0);  // uniform
    }
    // With four chunks or more, the next tile's metadata is fetched during
    // the chunk loop (its list entry after the barrier of step 1, the rest
    // after that of step 2, each waited for by the next step's vmcnt wait);
    // otherwise after the tile's extraction.
    const bool pf_loop = g.C / kChunk >= 4;
    for (int idx = __builtin_amdgcn_readfirstlane(next_tile); idx < hi;
         idx = __builtin_amdgcn_readfirstlane(next_tile)) {  // uniform
    int taken;  // thread 0 only
    if (threadIdx.x == 0) taken = atomicAdd(counter, 1);
    int nidx = hi;  // the next tile, once read (uniform)
    const int e = edge_of(idx);
    const int r = __builtin_amdgcn_readfirstlane(sm.pf_r);
    const int mt = r / ntiles, vt = r - mt * ntiles;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    const int HW = g.HW, Ttot = g.Ttot;
    const int p0 = mt * kSrcTile, v0 = vt * kTgtTile;
    const size_t plane = (size_t)g.C * Ttot;
    const unsigned short* fa = feat + (size_t)es.si[e] * slot_elems;
    const unsigned short* fb = feat + (size_t)es.sj[e] * slot_elems;
    // the rows' inverse split scales (powers of two), after the planes
    const float* isa = reinterpret_cast<const float*>(fa + 2 * plane);
    const float* isb = reinterpret_cast<const float*>(fb + 2 * plane);
    // the source tile's target boxes: virtual rows cum[l] .. cum[l + 1] - 1 are
    // level l's box (bh x bw cells from row ya, column xa), row-major
    int bya[kMaxLevels], bxa[kMaxLevels], bwd[kMaxLevels], cum[kMaxLevels + 1];
    {
        const int* rec = sm.pf_rec;
        cum[0] = 0;
#pragma unroll
        for (int l = 0; l < kMaxLevels; l++) {
            bya[l] = rec[4 * l];
            bxa[l] = rec[4 * l + 1];
            bwd[l] = rec[4 * l + 3];
            cum[l + 1] = cum[l] + rec[4 * l + 2] * bwd[l];
        }
    }
    const int total = cum[kMaxLevels];
    // target row (concatenated levels) of virtual row v; rows past the boxes
    // read row 0 (reaching accumulator cells never read), and every row is
    // clamped into the slot. (Each level's candidate is formed and the one
    // whose range holds v kept: a selection of the box fields by a computed
    // level would index them from memory.)
    auto trow = [&](int v) {
        int t = 0;
#pragma unroll
        for (int l = 0; l < kMaxLevels; l++) {
            const int r = v - cum[l];
            const int bw = std::max(bwd[l], 1);
            const int q = r / bw;
            const int c = g.off[l] + (bya[l] + q) * g.w[l] + bxa[l] + (r - q * bw);
            t = r >= 0 && v < cum[l + 1] ? c : t;
        }
        return std::min(std::max(t, 0), Ttot - 1);
    };

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
    const int pa = std::min((unsigned)sm.pf_pix[hr], (unsigned)(HW - 1));
    if (!(tid & 1)) sm.pix[hr] = pa;  // read after the chunk loop's barriers
    // wave (half, comp) stages coordinate comp (x, y) of sources half * 64 ..
    // + 63: gathered by their pixels (clamped like pa)
    const float* cpt = coords + ((size_t)e * 2 + (wave >> 1)) * HW +
                       std::min((unsigned)sm.pf_pix[(wave & 1) * 64 + lane], (unsigned)(HW - 1));
    const int tr0 = trow(v0 + hr), tr1 = trow(v0 + 128 + hr);
    // the inverse scales of source row hr and target rows hr, 128 + hr: loaded
    // ahead of the chunk loop's staging (whose waits count loads in issue
    // order) and put in LDS after it
    const float sc_a = isa[pa], sc_b0 = isb[tr0], sc_b1 = isb[tr1];
    const unsigned short* ga = fa + (size_t)pa * kChunk + hh;
    const unsigned short* gb0 = fb + (size_t)tr0 * kChunk + hh;
    const unsigned short* gb1 = fb + (size_t)tr1 * kChunk + hh;
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
            dma_x1(cpt, lds_addr(&sm.crd[comp][half * 64]));
        }
        if (nk > 1) issue(1, 1);
        // A wave's chunk loop issues at priority 1, its extraction (and the
        // next tile's set-up) at 2: on a SIMD shared with the other
        // workgroup's wave, the extraction's short dependent chains go first
        // and the MFMAs take the slots between them (measured ~1.5% faster
        // than the extraction at 0, which was ~1.5% faster than no
        // priorities).
        __builtin_amdgcn_s_setprio(1);
        for (int k = 0; k < nk; k++) {
            if (k + 1 < nk)
                __builtin_amdgcn_s_waitcnt(kWaitVm0Lgkm0 | kLoads);  // vmcnt(kLoads) lgkmcnt(0)
            else
                __builtin_amdgcn_s_waitcnt(kWaitVm0Lgkm0);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_barrier();
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            // the next tile: its index after every wave has read this one's
            // (step 0), its metadata loads older than the chunk loads they
            // are waited on with (steps 1 and 2)
            if (k == 0 && tid == 0) next_tile = lo + taken;
            if (pf_loop && k == 1) {  // uniform
                nidx = __builtin_amdgcn_readfirstlane(next_tile);
                if (nidx < hi) pf_list(nidx);
            }
            if (pf_loop && k == 2 && nidx < hi) pf_rest(nidx);
            if (k + 2 < nk) issue(k + 2, (k + 2) % kStages);
            compute(k % kStages);
        }
    };
    if constexpr (kF16) {
        // a target tile with a pooled row has lo planes (pooled fp16 values
        // are fp32 sums)
        const bool blo = alo || (cum[1] < total && v0 + kTgtTile > cum[1]);
        if (alo)
            chunk_loop(bool_c<true>{}, bool_c<true>{});
        else if (blo)
            chunk_loop(bool_c<false>{}, bool_c<true>{});
        else
            chunk_loop(bool_c<false>{}, bool_c<false>{});
    } else {
        chunk_loop(bool_c<true>{}, bool_c<true>{});
    }
    __builtin_amdgcn_s_setprio(2);
    if (tid < kSrcTile) {
        const bool in = p0 + tid < HW;
        sm.org[tid][0] = in ? floor_clamped(sm.crd[0][tid]) : -(1 << 20);  // matches no cell
        sm.org[tid][1] = in ? floor_clamped(sm.crd[1][tid]) : -(1 << 20);
    }
    if (!(tid & 1)) {
        sm.ssc[hr] = alpha * sc_a;  // powers of two: no rounding
        sm.tsc[hr] = sc_b0;
        sm.tsc[128 + hr] = sc_b1;
    }
    lds_barrier();  // every wave is done with the stages before T overwrites them

    // ---- window extraction ----
    // whether this tile holds virtual rows of level l's box
    bool lin[kMaxLevels];
#pragma unroll
    for (int l = 0; l < kMaxLevels; l++)
        lin[l] = cum[l + 1] > cum[l] && cum[l] < v0 + kTgtTile && cum[l + 1] > v0;
    // accumulator layout of the 32x32 MFMA: lane l, register v holds
    // D[i][j] with j = l % 32 (target) and i = 8*(v/4) + 4*(l/32) + v%4 (source)
    const int khalf = lane >> 5;
    // extraction: a wave takes its 16 columns of T (sources); lane = (source jj,
    // quarter qq), and in each of 4 rounds a lane reads 4 consecutive cells of
    // one window row (cells 4 * (f & 1) .. +3 of row f >> 1, f = 4 * round +
    // qq) and stores them with one 16-byte store, so a store instruction covers
    // 16 sources x 4 quarter-rows.
    const int jj = lane >> 2, qq = lane & 3;
    // Window stores go through a buffer resource over this edge's window slot:
    // a lane with nothing to store gets an offset past the slot's size, and
    // the hardware discards the store, so store instructions are issued
    // without a branch around them. A 4-cell piece is stored whole by the one
    // tile holding all of its in-grid cells (the cells outside the grid are
    // never read: the lookup zeroes them); a piece whose in-grid cells a
    // virtual-tile boundary splits is stored cell by cell by both tiles.
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        win + win_index(slot0 + e, 0, 0, HW, 0), 0, kMaxLevels * 64 * HW * (int)sizeof(float),
        kBufWord3);
    typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

    // T holds the accumulators times their targets' inverse scales (powers of
    // two: no rounding); the extraction multiplies by alpha times the
    // source's, so each cell is rounded once, as alpha times its fp32 sum
    float tsv[4];
#pragma unroll
    for (int tb = 0; tb < 4; tb++) tsv[tb] = sm.tsc[wn * 128 + tb * 32 + orow];
#pragma unroll
    for (int sb = 0; sb < 2; sb++) {
        if (sb) lds_barrier();  // the first half's cells have all been read
#pragma unroll
        for (int tb = 0; tb < 4; tb++)
#pragma unroll
            for (int gq = 0; gq < 4; gq++) {
                const int t = wn * 128 + tb * 32 + orow;
                const int s = wm * 32 + gq * 8 + khalf * 4;
                *reinterpret_cast<float4*>(&sm.u.T[kTPad + t][s]) = make_float4(
                    acc[sb][tb][4 * gq] * tsv[tb], acc[sb][tb][4 * gq + 1] * tsv[tb],
                    acc[sb][tb][4 * gq + 2] * tsv[tb], acc[sb][tb][4 * gq + 3] * tsv[tb]);
            }
        lds_barrier();
        const int s = wave * 16 + jj;                            // column of T
        const int lsrc = (s >> 5) * 64 + sb * 32 + (s & 31);   // source in the tile
        const int fx = sm.org[lsrc][0], fy = sm.org[lsrc][1];
        const float fs = sm.ssc[lsrc];
        const bool pin = p0 + lsrc < HW;
        // column s of T at target row 0 (rows -kTPad .. kTgtTile + kTPad - 1 exist)
        const float* Tcol = &sm.u.T[kTPad][s];
        // byte offset of cell 0 of row 0 of level 0 of this source in the slot
        const int woff = (int)win_index(0, 0, 0, HW, sm.pix[lsrc]) * 4;
        // the lane's pieces: window rows 2 rd + cyq (rounds rd = 0..3), cells
        // cx0 .. cx0 + 3 of each
        const int cyq = qq >> 1, cx0 = (qq & 1) * 4;
#pragma unroll
        for (int l = 0; l < kMaxLevels; l++) {
            if (!lin[l]) continue;  // level not in this tile
            const int hl = g.h[l], bw = bwd[l];
            const int x0 = (fx >> l) - 3 + cx0, y0 = (fy >> l) - 3 + cyq;
            // the piece's in-grid cells are ia..ib (the same in every round);
            // tile row of its first cell in round 0, 2 bw further each round
            // (every in-grid cell of the tile's windows lies in the box; the
            // value is meaningless, and unused, for rows outside the grid)
            const int ia = std::max(0, -x0), ib = std::min(3, g.w[l] - 1 - x0);
            const bool xok = pin && ia <= ib;
            const unsigned t00 = (unsigned)(cum[l] - v0) + (unsigned)(y0 - bya[l]) * (unsigned)bw +
                                 (unsigned)(x0 - bxa[l]);
            int tl[4];
            bool has[4], full[4];
            float v[4][4];
            // every round's reads go out before the first store: a piece with
            // an in-grid cell in the tile has tl in [-kTPad, kTgtTile - 1], so
            // its four rows lie in T; another reads row 0
#pragma unroll
            for (int rd = 0; rd < 4; rd++) {
                tl[rd] = (int)(t00 + (unsigned)(2 * rd * bw));
                const int ta = tl[rd] + ia, tb = tl[rd] + ib;
                // some in-grid cell in this tile; all of them
                has[rd] = xok && (unsigned)(y0 + 2 * rd) < (unsigned)hl && ta < kTgtTile && tb >= 0;
                full[rd] = has[rd] && ta >= 0 && tb < kTgtTile;
                const float* tp = Tcol + (has[rd] ? tl[rd] : 0) * kTStride;
#pragma unroll
                for (int i = 0; i < 4; i++) v[rd][i] = tp[i * kTStride];
            }
#pragma unroll
            for (int rd = 0; rd < 4; rd++) {
                const int off = woff + ((l * 8 + cyq + 2 * rd) * HW * 8 + cx0) * 4;
                const u32x4_t pk = {__builtin_bit_cast(unsigned, fs * v[rd][0]),
                                    __builtin_bit_cast(unsigned, fs * v[rd][1]),
                                    __builtin_bit_cast(unsigned, fs * v[rd][2]),
                                    __builtin_bit_cast(unsigned, fs * v[rd][3])};
                __builtin_amdgcn_raw_buffer_store_b128(pk, wrs, full[rd] ? off : kBufDiscard, 0,
                                                       0);
                const bool split = has[rd] && !full[rd];
                if (__ballot(split)) {  // uniform, rare: a piece cut by the tile's ends
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const bool val = split && i >= ia && i <= ib &&
                                         (unsigned)(tl[rd] + i) < (unsigned)kTgtTile;
                        __builtin_amdgcn_raw_buffer_store_b32(pk[i], wrs,
                                                              val ? off + 4 * i : kBufDiscard, 0,
                                                              0);
                    }
                }
            }
        }
    }
    lds_barrier();  // T is free again, next_tile is visible
    if (!pf_loop) {
        const int n = __builtin_amdgcn_readfirstlane(next_tile);
        if (n < hi) pf_sync(n);  // uniform
    }
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
// each row's inverse split scale (Ttot floats), padded to 256 bytes
size_t slot_elems(const Geom& g) {
    return (2 * (size_t)g.C * g.Ttot + 2 * (size_t)g.Ttot + 127) / 128 * 128;
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
    const int nbx = (g.w[0] + kPW - 1) / kPW;
    const int nblk = nbx * ((g.h[0] + kPH - 1) / kPH);
    const long nprep = (long)nblk * std::max(nslots, 0);
    const long nmask = mk.list ? mk.nedges : 0;
    if (nprep + nmask == 0) return SLK_OK;
    if (nprep + nmask > INT_MAX) return fail(SLK_E_ARG, "feature preparation grid too large");
    if (g.C > kPrepC) return fail(SLK_E_ARG, "feature preparation: more than 128 channels");
    const long se = (long)slot_elems(g);
    ProfScope ps(ctx, "corr_feat_prep", stream);
    hipLaunchKernelGGL((k_feat_prep<Tin>), dim3((unsigned)(nprep + nmask)), dim3(1024), 0, stream,
                       fm, fstride, sf, slot_lo, out, se, g, pooled ? 1 : 0, nbx, nblk,
                       (int)nmask, mk, mode);
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

// The order workgroups (with the preparation of nslots slots when
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
    const KeyGeom kg = key_geom(g);
    if (kg.nkeys > kMaxKeys) return fail(SLK_E_ARG, "correlation: map too tall for the source sort");
    if (mtiles > kPrepL1Words)
        return fail(SLK_E_ARG, "correlation: more source tiles per edge than the order pass holds");
    const long ostride = order_stride(g.HW, mtiles);
    MaskArgs mk{coords, ctx->tile_list.as<int>(), ctx->tile_ctr.as<int>(),
                ctx->src_order.as<int>(), ostride, mtiles, ntiles, n, kg};
    // feature preparation and the source order, one launch
    SLK_TRY(prep_slots(ctx, fm, fstride, sf, g, slot_lo, nslots, pooled, mk, mode, stream));
    {
        ProfScope ps(ctx, "corr_window", stream);
        const long se = (long)slot_elems(g);
        if (mode == kSplitF16)
            hipLaunchKernelGGL(k_corr_split_win<true>, dim3(ctx->ws_grid), dim3(256), 0, stream,
                               feat, se, es, ctx->src_order.as<int>(), ostride, coords, win,
                               slot0, g,
                               ctx->alpha, mtiles, ntiles, n, ctx->tile_list.as<int>(),
                               ctx->tile_ctr.as<int>(), alo ? 1 : 0);
        else
            hipLaunchKernelGGL(k_corr_split_win<false>, dim3(ctx->ws_grid), dim3(256), 0, stream,
                               feat, se, es, ctx->src_order.as<int>(), ostride, coords, win,
                               slot0, g,
                               ctx->alpha, mtiles, ntiles, n, ctx->tile_list.as<int>(),
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
        const MaskArgs none{};
        SLK_TRY(prep_slots(ctx, fm, fstride, sf, g, 0, n, false, none, mode, stream));
    }
    return mask_and_windows(ctx, fm, fstride, sf, g, n, n, true, es, feat, n, coords, win, slot0,
                            mode, alo, stream);
}

}  // namespace

// the split path: whole 16-channel chunks, at most kPrepC channels (a
// preparation block holds all of a pixel's), and an edge's source tiles within
// the order pass's LDS (h*w <= 262144); other maps take the fp32 MFMA kernels
bool corr_split_supported(const slk_ctx* ctx) {
    return ctx->C % kChunk == 0 && ctx->C <= kPrepC &&
           (ctx->HW + kSrcTile - 1) / kSrcTile <= kPrepL1Words;
}

void corr_split_footprint(const slk_ctx* ctx, size_t* slot_bytes, size_t* tiles_per_edge,
                          size_t* order_per_edge, size_t* ctr_bytes) {
    const Geom g = make_geom(ctx);
    const size_t mtiles = (g.HW + kSrcTile - 1) / kSrcTile;
    const size_t ntiles = (g.Ttot + kTgtTile - 1) / kTgtTile;
    *slot_bytes = slot_elems(g) * sizeof(unsigned short);
    *tiles_per_edge = mtiles * ntiles * sizeof(int);
    *order_per_edge = (size_t)order_stride(g.HW, (int)mtiles) * sizeof(int);
    *ctr_bytes = kCtrInts * sizeof(int);
}

int corr_split_grid(int cus) { return std::max(8, cus / 8 * 8) * 2; }

int corr_split_alloc(slk_ctx* ctx) {
    if (!corr_split_supported(ctx)) return SLK_OK;
    const Geom g = make_geom(ctx);
    const size_t slots = 2 * (size_t)std::min(ctx->max_batch, kMaxEdgesPerLaunch);
    SLK_TRY(ctx->split_feat.ensure(slots * slot_elems(g) * sizeof(unsigned short)));
    const size_t mtiles = (g.HW + kSrcTile - 1) / kSrcTile;
    const size_t ntiles = (g.Ttot + kTgtTile - 1) / kTgtTile;
    const size_t tiles = (size_t)std::min(ctx->max_batch, kMaxEdgesPerLaunch) * mtiles * ntiles;
    SLK_TRY(ctx->tile_list.ensure(tiles * sizeof(int)));
    SLK_TRY(ctx->src_order.ensure((size_t)std::min(ctx->max_batch, kMaxEdgesPerLaunch) *
                                  order_stride(g.HW, (int)mtiles) * sizeof(int)));
    SLK_TRY(ctx->tile_ctr.ensure(kCtrInts * sizeof(int)));
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
    SlotFrames sf{};
    sf.ident = 1;
    const MaskArgs none{};
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
