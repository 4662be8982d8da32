// All-pairs correlation, 2x2 average-pool pyramid and radius-3 bilinear
// lookup for gfx950 (MI355X).
//
// Reference semantics: cuda_slam/main.cu:1077-1217 (kernels) and :1500-1613
// (build_correlation, sample_correlation, batch_build_and_sample_correlation).
//
// k_corr_tile: vol[e][p][q] = alpha * sum_c fa[c][p] * fb[c][q] on fp32 MFMA
// (v_mfma_f32_32x32x2f32), with every pyramid level produced in the epilogue
// from the tile still in registers. A workgroup is 4 waves stacked over 4x32
// source pixels; each wave owns an 8-row x 32-column band of the target image
// (eight 32x32 accumulator blocks), which is exactly one group of level-3
// cells, so levels 1..3 never need data from another wave: x-pairs come from
// the neighbouring lane (lane ^ 1, ^ 2, ^ 4), y-pairs from the accumulator
// block of the next target row. Operands are read straight from global memory
// in the MFMA operand layout (consecutive lanes = consecutive pixels of one
// channel: 128-byte coalesced per half-wave), double-buffered in registers so
// the next 8 channels are in flight while the MFMAs of the current 8 run.
//
// Two epilogues:
//   * materializing (single-edge build_correlation): every level is stored in
//     the reference's layout [HW][h>>l][w>>l] (debug dump, sample_correlation);
//   * windowed (batched build_and_sample): the caller never sees the volume,
//     so each tile stores only the cells that fall in some source pixel's 8x8
//     lookup window at that level, into a compact [HW][levels][8][8] buffer.
//     The volume and pyramid (~50 MB per 48x64 edge) never reach HBM; the
//     windows are 1 KB per source pixel.
#include <algorithm>
#include <cmath>
#include <mutex>
#include <type_traits>

#include "corr_common.hpp"

namespace slk {
namespace {

constexpr int kWG = 256;           // 4 waves
constexpr int kWaveSrc = 32;       // source pixels per wave
constexpr int kTileSrc = 128;      // source pixels per workgroup
constexpr int kBand = 8;           // target rows per tile (2^(levels-1) for 4 levels)
constexpr int kCols = 32;          // target columns per tile
constexpr int kKU = 4;             // 2-channel MFMA steps per prefetch group

struct EdgeIdx {
    int ii[kMaxEdgesPerLaunch];
    int jj[kMaxEdgesPerLaunch];
};

struct LevelOut {
    float* p[kMaxLevels];
};

__device__ __forceinline__ float ldf(const float* p) { return *p; }
__device__ __forceinline__ float ldf(const _Float16* p) { return (float)(*p); }

// Operands of kKU 2-channel steps. Lanes of sources past HW or targets outside
// the image read a clamped in-bounds address instead of being zeroed: an MFMA
// output D[i][j] only combines row i of A with column j of B, so such lanes
// only reach accumulator rows/columns that are never stored, and never a
// stored pooled cell (a pooled cell inside the level only averages targets
// inside the image). Leaving the values unselected lets the loads stay in
// flight under the previous group's MFMAs.
template <typename Tin>
__device__ __forceinline__ void load_group(const Tin* A, const Tin* Bp, const int* boff, long HW,
                                           int c0, float* a, float (*b)[kBand]) {
#pragma unroll
    for (int u = 0; u < kKU; u++) {
        const long off = (long)(c0 + 2 * u) * HW;
        a[u] = ldf(A + off);
#pragma unroll
        for (int r = 0; r < kBand; r++) b[u][r] = ldf(Bp + off + boff[r]);
    }
}

template <typename Tin, bool WIN>
__global__ __launch_bounds__(kWG) void k_corr_tile(
    const Tin* __restrict__ fa, const Tin* __restrict__ fb, long fstride,
    const int* __restrict__ ia, const int* __restrict__ ib, EdgeIdx eidx, LevelOut lo,
    const float* __restrict__ coords, float* __restrict__ win, int slot0, int h, int w, int C,
    float alpha, int levels, int mtiles, int nbands, int ncb) {
    const int HW = h * w;
    const int tpe = mtiles * nbands * ncb;
    const int bid = xcd_remap(blockIdx.x, gridDim.x);
    const int e = bid / tpe;
    int t = bid - e * tpe;
    const int cb = t % ncb;
    t /= ncb;
    const int band = t % nbands;
    const int mt = t / nbands;

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int p0 = mt * kTileSrc + wave * kWaveSrc;
    if (p0 >= HW) return;  // whole wave outside (no LDS, no barriers)
    const int y0 = band * kBand, x0 = cb * kCols;
    const int col = lane & 31, khalf = lane >> 5;

    const int fi = ia ? ia[e] : eidx.ii[e];
    const int fj = ib ? ib[e] : eidx.jj[e];
    const int pa = p0 + col;
    const bool va = pa < HW;
    const Tin* A = fa + (long)fi * fstride + (long)khalf * HW + (va ? pa : 0);
    const int xb = x0 + col;
    const Tin* Bp = fb + (long)fj * fstride + (long)khalf * HW;
    int boff[kBand];
    bool vb[kBand];
#pragma unroll
    for (int r = 0; r < kBand; r++) {
        const int y = y0 + r;
        vb[r] = (y < h) && (xb < w);
        boff[r] = vb[r] ? y * w + xb : 0;
    }

    f32x16 acc[kBand];
#pragma unroll
    for (int r = 0; r < kBand; r++) acc[r] = (f32x16){0};

    // main loop: groups of kKU 2-channel steps, next group loaded before the
    // current group's MFMAs are issued
    // Two register sets used in ping-pong (no copies, which would make every
    // group wait for its own loads).
    const int ngroups = C / (2 * kKU);
    float a0[kKU], b0[kKU][kBand], a1[kKU], b1[kKU][kBand];
    auto mfma_group = [&](const float* a, const float (*b)[kBand]) {
#pragma unroll
        for (int u = 0; u < kKU; u++)
#pragma unroll
            for (int r = 0; r < kBand; r++)
                acc[r] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[u], b[u][r], acc[r], 0, 0, 0);
    };
    if (ngroups > 0) load_group(A, Bp, boff, HW, 0, a0, b0);
    for (int g = 0; g < ngroups; g += 2) {
        if (g + 1 < ngroups) load_group(A, Bp, boff, HW, (g + 1) * 2 * kKU, a1, b1);
        mfma_group(a0, b0);
        if (g + 2 < ngroups) load_group(A, Bp, boff, HW, (g + 2) * 2 * kKU, a0, b0);
        if (g + 1 < ngroups) mfma_group(a1, b1);
    }
    for (int c = ngroups * 2 * kKU; c < C; c += 2) {  // C not a multiple of 2*kKU
        const long off = (long)c * HW;
        const float a = ldf(A + off);
#pragma unroll
        for (int r = 0; r < kBand; r++)
            acc[r] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, ldf(Bp + off + boff[r]), acc[r], 0,
                                                          0, 0);
    }

    // Accumulator layout of v_mfma_f32_32x32x2f32: lane l, register v holds
    // D[i][j] with j = l % 32 (target column) and
    // i = 8*(v/4) + 4*(l/32) + v%4 (source row of the wave's 32).
    const int slot = slot0 + e;
#pragma unroll
    for (int r = 0; r < kBand; r++) {
#pragma unroll
        for (int v = 0; v < 16; v++) acc[r][v] *= alpha;
    }
    int prow[16];
#pragma unroll
    for (int v = 0; v < 16; v++) prow[v] = p0 + 8 * (v >> 2) + 4 * khalf + (v & 3);
    float cxs[16], cys[16];
    if constexpr (WIN) {
        const float* cc = coords + (size_t)e * 2 * HW;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int q = prow[v] < HW ? prow[v] : 0;
            cxs[v] = cc[q];
            cys[v] = cc[HW + q];
        }
    }
    // store of one cell (y, x) of level l for source row register v
    auto put = [&](int l, int v, int y, int x, float val, float* plane, int hl, int wl) {
        const int p = prow[v];
        if (p >= HW) return;
        if constexpr (WIN) {
            const int ox = x - win_origin(cxs[v], l);
            const int oy = y - win_origin(cys[v], l);
            if ((unsigned)ox < 8u && (unsigned)oy < 8u)
                win[win_index(slot, l, oy * 8 + ox, HW, p)] = val;
        } else {
            __builtin_nontemporal_store(val, plane + (size_t)p * (hl * wl) + y * wl + x);
        }
    };

    float* out0 = WIN ? nullptr : lo.p[0] + (size_t)slot * HW * HW;
#pragma unroll
    for (int r = 0; r < kBand; r++) {
        if (!vb[r]) continue;
#pragma unroll
        for (int v = 0; v < 16; v++) put(0, v, y0 + r, xb, acc[r][v], out0, h, w);
    }
    if (levels < 2) return;

    // level 1: 0.25f*(((in[y][x] + in[y][x+1]) + in[y+1][x]) + in[y+1][x+1]),
    // the order of avg_pool_2x2_kernel (main.cu:1166-1167)
    const int h1 = h >> 1, w1 = w >> 1;
    float l1[4][16];
#pragma unroll
    for (int r = 0; r < 4; r++) {
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const float a = acc[2 * r][v];
            const float c = acc[2 * r + 1][v];
            const float b = __shfl_xor(a, 1);
            const float d = __shfl_xor(c, 1);
            float s = a + b;
            s = s + c;
            s = s + d;
            l1[r][v] = 0.25f * s;
        }
    }
    {
        float* out1 = WIN ? nullptr : lo.p[1] + (size_t)slot * HW * (h1 * w1);
        const int x1 = xb >> 1;
        const bool lane_ok = ((col & 1) == 0) && x1 < w1;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int y1 = (y0 >> 1) + r;
            if (!lane_ok || y1 >= h1) continue;
#pragma unroll
            for (int v = 0; v < 16; v++) put(1, v, y1, x1, l1[r][v], out1, h1, w1);
        }
    }
    if (levels < 3) return;

    const int h2 = h >> 2, w2 = w >> 2;
    float l2[2][16];
#pragma unroll
    for (int r = 0; r < 2; r++) {
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const float a = l1[2 * r][v];
            const float c = l1[2 * r + 1][v];
            const float b = __shfl_xor(a, 2);
            const float d = __shfl_xor(c, 2);
            float s = a + b;
            s = s + c;
            s = s + d;
            l2[r][v] = 0.25f * s;
        }
    }
    {
        float* out2 = WIN ? nullptr : lo.p[2] + (size_t)slot * HW * (h2 * w2);
        const int x2 = xb >> 2;
        const bool lane_ok = ((col & 3) == 0) && x2 < w2;
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int y2 = (y0 >> 2) + r;
            if (!lane_ok || y2 >= h2) continue;
#pragma unroll
            for (int v = 0; v < 16; v++) put(2, v, y2, x2, l2[r][v], out2, h2, w2);
        }
    }
    if (levels < 4) return;

    const int h3 = h >> 3, w3 = w >> 3;
    float* out3 = WIN ? nullptr : lo.p[3] + (size_t)slot * HW * (h3 * w3);
    const int x3 = xb >> 3, y3 = y0 >> 3;
    const bool lane_ok = ((col & 7) == 0) && x3 < w3 && y3 < h3;
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const float a = l2[0][v];
        const float c = l2[1][v];
        const float b = __shfl_xor(a, 4);
        const float d = __shfl_xor(c, 4);
        float s = a + b;
        s = s + c;
        s = s + d;
        if (lane_ok) put(3, v, y3, x3, 0.25f * s, out3, h3, w3);
    }
}

// ------------------------------------------ split-precision MFMA kernel --
// k_corr_mx: same tile, pyramid and epilogues as k_corr_tile, with the
// contraction on the 16-wide-K matrix instructions of gfx950:
//   fp32 features: each value is split into bf16 hi + lo (hi = rne(x),
//     lo = rne(x - hi)) and vol = hi.hi + hi.lo + lo.hi on
//     v_mfma_f32_32x32x16_bf16 (exact products, fp32 accumulation; the
//     dropped lo.lo term and the rounding of lo are ~2^-16 relative per
//     product) -- fp32-grade accuracy at 16x the fp32 MFMA rate, 3 passes;
//   fp16 features: one v_mfma_f32_32x32x16_f16 pass (exact products, fp32
//     accumulation: the arithmetic of the reference's cublasGemmEx on its
//     fp16 fmaps, main.cu:1508-1515).
// Operands are staged through LDS in 16-channel chunks, double-buffered: each
// chunk is read once from global memory per workgroup, converted once, and
// the global loads of chunk k+1 are in flight during the MFMAs of chunk k.
// LDS rows are 48 bytes (16 values + pad) so the 128-bit operand reads of a
// 32x32x16 MFMA (lane l: row l%32, 8 consecutive k at 8*(l/32)) hit
// distinct banks. Waves form a 2x2 grid over the workgroup's 128 sources x
// 8 target rows: wave (wm, wn) owns sources wm*64..+63 and rows wn*4..+3
// (eight 32x32 accumulator blocks); level 3 pools across the two row halves
// through LDS.

constexpr int kKC = 16;        // channels per LDS stage
constexpr int kRowU = 24;      // u16 per LDS operand row (16 used + 8 pad)
constexpr int kTileTgt = 256;  // targets per workgroup tile (8 rows x 32 cols)
enum { kModeBF16x3 = 0, kModeF16 = 1 };

template <int MODE>
struct MxSmem {
    static constexpr int NP = MODE == kModeBF16x3 ? 2 : 1;  // hi (+ lo)
    unsigned short A[2][NP][kTileSrc][kRowU];
    unsigned short B[2][NP][kTileTgt][kRowU];
};

template <int MODE>
__device__ __forceinline__ f32x16 mfma16(u16x8_t a, u16x8_t b, f32x16 c) {
    if constexpr (MODE == kModeBF16x3)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0,
                                                       0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                      __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

template <int MODE, bool WIN>
__global__ __launch_bounds__(kWG) void k_corr_mx(
    const void* __restrict__ fa_, const void* __restrict__ fb_, long fstride,
    const int* __restrict__ ia, const int* __restrict__ ib, EdgeIdx eidx, LevelOut lo,
    const float* __restrict__ coords, float* __restrict__ win, int slot0, int h, int w, int C,
    float alpha, int levels, int mtiles, int nbands, int ncb) {
    using Tin = typename std::conditional<MODE == kModeBF16x3, float, _Float16>::type;
    constexpr int NP = MxSmem<MODE>::NP;
    __shared__ MxSmem<MODE> sm;
    const int HW = h * w;
    const int tpe = mtiles * nbands * ncb;
    const int bid = xcd_remap(blockIdx.x, gridDim.x);
    const int e = bid / tpe;
    int t = bid - e * tpe;
    const int cb = t % ncb;
    t /= ncb;
    const int band = t % nbands;
    const int mt = t / nbands;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave & 1, wn = wave >> 1;
    const int y0 = band * kBand, x0 = cb * kCols;
    const int fi = ia ? ia[e] : eidx.ii[e];
    const int fj = ib ? ib[e] : eidx.jj[e];
    const Tin* Ab = static_cast<const Tin*>(fa_) + (long)fi * fstride;
    const Tin* Bb = static_cast<const Tin*>(fb_) + (long)fj * fstride;

    // staging roles: A -- source tid%128, channels (tid/128)*8..+7 of the
    // chunk; B -- target tid (row tid/32, column tid%32), all 16 channels.
    // Out-of-range pixels read a clamped address (see load_group).
    const int a_src = tid & (kTileSrc - 1), a_half = tid >> 7;
    const int pa = mt * kTileSrc + a_src;
    const Tin* a_ptr = Ab + (long)(a_half * 8) * HW + (pa < HW ? pa : 0);
    const int by = y0 + (tid >> 5), bx = x0 + (tid & 31);
    const Tin* b_ptr = Bb + ((by < h && bx < w) ? by * w + bx : 0);
    Tin ra[8], rb[kKC];
    auto gload = [&](int c0) {
#pragma unroll
        for (int u = 0; u < 8; u++) ra[u] = a_ptr[(long)(c0 + u) * HW];
#pragma unroll
        for (int u = 0; u < kKC; u++) rb[u] = b_ptr[(long)(c0 + u) * HW];
    };
    auto lstore = [&](int st) {
        u16x8_t hi, lo8;
        if constexpr (MODE == kModeBF16x3) {
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const unsigned s = split_bf16(ra[u]);
                hi[u] = (unsigned short)(s & 0xffffu);
                lo8[u] = (unsigned short)(s >> 16);
            }
            *reinterpret_cast<u16x8_t*>(&sm.A[st][0][a_src][a_half * 8]) = hi;
            *reinterpret_cast<u16x8_t*>(&sm.A[st][1][a_src][a_half * 8]) = lo8;
#pragma unroll
            for (int half = 0; half < 2; half++) {
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const unsigned s = split_bf16(rb[half * 8 + u]);
                    hi[u] = (unsigned short)(s & 0xffffu);
                    lo8[u] = (unsigned short)(s >> 16);
                }
                *reinterpret_cast<u16x8_t*>(&sm.B[st][0][tid][half * 8]) = hi;
                *reinterpret_cast<u16x8_t*>(&sm.B[st][1][tid][half * 8]) = lo8;
            }
        } else {
#pragma unroll
            for (int u = 0; u < 8; u++) hi[u] = __builtin_bit_cast(unsigned short, ra[u]);
            *reinterpret_cast<u16x8_t*>(&sm.A[st][0][a_src][a_half * 8]) = hi;
#pragma unroll
            for (int half = 0; half < 2; half++) {
#pragma unroll
                for (int u = 0; u < 8; u++)
                    hi[u] = __builtin_bit_cast(unsigned short, rb[half * 8 + u]);
                *reinterpret_cast<u16x8_t*>(&sm.B[st][0][tid][half * 8]) = hi;
            }
        }
    };

    f32x16 acc[2][4];
#pragma unroll
    for (int sb = 0; sb < 2; sb++)
#pragma unroll
        for (int tb = 0; tb < 4; tb++) acc[sb][tb] = (f32x16){0};
    const int orow = lane & 31, okk = (lane >> 5) * 8;
    auto compute = [&](int st) {
        u16x8_t ah[2], al[2], bh[4], bl[4];
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
            ah[sb] = *reinterpret_cast<const u16x8_t*>(&sm.A[st][0][wm * 64 + sb * 32 + orow][okk]);
            if constexpr (NP == 2)
                al[sb] =
                    *reinterpret_cast<const u16x8_t*>(&sm.A[st][NP - 1][wm * 64 + sb * 32 + orow][okk]);
        }
#pragma unroll
        for (int tb = 0; tb < 4; tb++) {
            bh[tb] = *reinterpret_cast<const u16x8_t*>(&sm.B[st][0][(wn * 4 + tb) * 32 + orow][okk]);
            if constexpr (NP == 2)
                bl[tb] = *reinterpret_cast<const u16x8_t*>(
                    &sm.B[st][NP - 1][(wn * 4 + tb) * 32 + orow][okk]);
        }
        if constexpr (MODE == kModeBF16x3) {
            // small cross terms first, then hi.hi; eight independent
            // accumulators between dependent MFMAs
#pragma unroll
            for (int sb = 0; sb < 2; sb++)
#pragma unroll
                for (int tb = 0; tb < 4; tb++)
                    acc[sb][tb] = mfma16<MODE>(al[sb], bh[tb], acc[sb][tb]);
#pragma unroll
            for (int sb = 0; sb < 2; sb++)
#pragma unroll
                for (int tb = 0; tb < 4; tb++)
                    acc[sb][tb] = mfma16<MODE>(ah[sb], bl[tb], acc[sb][tb]);
        }
#pragma unroll
        for (int sb = 0; sb < 2; sb++)
#pragma unroll
            for (int tb = 0; tb < 4; tb++) acc[sb][tb] = mfma16<MODE>(ah[sb], bh[tb], acc[sb][tb]);
    };

    const int nchunks = C / kKC;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int ch = 0; ch < nchunks; ch++) {
        if (ch + 1 < nchunks) gload((ch + 1) * kKC);
        compute(ch & 1);
        if (ch + 1 < nchunks) lstore((ch + 1) & 1);
        __syncthreads();
    }

    // ---- epilogue (accumulator layout as in k_corr_tile) ----
    const int slot = slot0 + e;
    const int col = lane & 31, khalf = lane >> 5, xb = x0 + col;
    const int ps0 = mt * kTileSrc + wm * 64;
#pragma unroll
    for (int sb = 0; sb < 2; sb++)
#pragma unroll
        for (int tb = 0; tb < 4; tb++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[sb][tb][v] *= alpha;
    auto prow = [&](int sb, int v) { return ps0 + sb * 32 + 8 * (v >> 2) + 4 * khalf + (v & 3); };
    // coordinates of the lane's 32 source rows, loaded once before any store
    // (the window stores would otherwise order every later coordinate load)
    float cxs[2][16], cys[2][16];
    if constexpr (WIN) {
        const float* cc = coords + (size_t)e * 2 * HW;
#pragma unroll
        for (int sb = 0; sb < 2; sb++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int p = prow(sb, v);
                const int q = p < HW ? p : 0;
                cxs[sb][v] = cc[q];
                cys[sb][v] = cc[HW + q];
            }
    }
    auto put = [&](int l, int sb, int v, int y, int x, float val, float* plane, int hl, int wl) {
        const int p = prow(sb, v);
        if (p >= HW) return;
        if constexpr (WIN) {
            const int ox = x - win_origin(cxs[sb][v], l);
            const int oy = y - win_origin(cys[sb][v], l);
            if ((unsigned)ox < 8u && (unsigned)oy < 8u)
                win[win_index(slot, l, oy * 8 + ox, HW, p)] = val;
        } else {
            __builtin_nontemporal_store(val, plane + (size_t)p * (hl * wl) + y * wl + x);
        }
    };
    const int yw = y0 + wn * 4;  // first target row of this wave
    {
        float* out0 = WIN ? nullptr : lo.p[0] + (size_t)slot * HW * HW;
#pragma unroll
        for (int tb = 0; tb < 4; tb++) {
            const int y = yw + tb;
            if (y >= h || xb >= w) continue;
#pragma unroll
            for (int sb = 0; sb < 2; sb++)
#pragma unroll
                for (int v = 0; v < 16; v++) put(0, sb, v, y, xb, acc[sb][tb][v], out0, h, w);
        }
    }
    float l2[2][16];
    if (levels >= 2) {
        const int h1 = h >> 1, w1 = w >> 1, x1 = xb >> 1;
        float* out1 = WIN ? nullptr : lo.p[1] + (size_t)slot * HW * (h1 * w1);
        float l1[2][2][16];
#pragma unroll
        for (int sb = 0; sb < 2; sb++)
#pragma unroll
            for (int r = 0; r < 2; r++)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    // 0.25f*(((in[y][x] + in[y][x+1]) + in[y+1][x]) + in[y+1][x+1]),
                    // the order of avg_pool_2x2_kernel (main.cu:1166-1167)
                    const float a = acc[sb][2 * r][v], c = acc[sb][2 * r + 1][v];
                    const float b = __shfl_xor(a, 1), d = __shfl_xor(c, 1);
                    float s = a + b;
                    s = s + c;
                    s = s + d;
                    l1[sb][r][v] = 0.25f * s;
                }
        const bool ok1 = ((col & 1) == 0) && x1 < w1;
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int y1 = (yw >> 1) + r;
            if (!ok1 || y1 >= h1) continue;
#pragma unroll
            for (int sb = 0; sb < 2; sb++)
#pragma unroll
                for (int v = 0; v < 16; v++) put(1, sb, v, y1, x1, l1[sb][r][v], out1, h1, w1);
        }
        if (levels >= 3) {
            const int h2 = h >> 2, w2 = w >> 2, x2 = xb >> 2, y2 = yw >> 2;
            float* out2 = WIN ? nullptr : lo.p[2] + (size_t)slot * HW * (h2 * w2);
#pragma unroll
            for (int sb = 0; sb < 2; sb++)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const float a = l1[sb][0][v], c = l1[sb][1][v];
                    const float b = __shfl_xor(a, 2), d = __shfl_xor(c, 2);
                    float s = a + b;
                    s = s + c;
                    s = s + d;
                    l2[sb][v] = 0.25f * s;
                }
            if (((col & 3) == 0) && x2 < w2 && y2 < h2) {
#pragma unroll
                for (int sb = 0; sb < 2; sb++)
#pragma unroll
                    for (int v = 0; v < 16; v++) put(2, sb, v, y2, x2, l2[sb][v], out2, h2, w2);
            }
        }
    }
    if (levels >= 4) {
        // level-2 rows 2*y3 (waves wn = 0) and 2*y3 + 1 (wn = 1) meet in LDS
        float* xch = reinterpret_cast<float*>(&sm);  // [wm][sb][v][lane], 16 KB
        if (wn == 1) {
#pragma unroll
            for (int sb = 0; sb < 2; sb++)
#pragma unroll
                for (int v = 0; v < 16; v++) xch[((wm * 2 + sb) * 16 + v) * 64 + lane] = l2[sb][v];
        }
        __syncthreads();
        if (wn == 0) {
            const int h3 = h >> 3, w3 = w >> 3, x3 = xb >> 3, y3 = y0 >> 3;
            float* out3 = WIN ? nullptr : lo.p[3] + (size_t)slot * HW * (h3 * w3);
            const bool ok3 = ((col & 7) == 0) && x3 < w3 && y3 < h3;
#pragma unroll
            for (int sb = 0; sb < 2; sb++)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const float a = l2[sb][v];
                    const float b = __shfl_xor(a, 4);
                    const float* xr = xch + ((wm * 2 + sb) * 16 + v) * 64;
                    const float c = xr[lane], d = xr[lane ^ 4];
                    float s = a + b;
                    s = s + c;
                    s = s + d;
                    if (ok3) put(3, sb, v, y3, x3, 0.25f * s, out3, h3, w3);
                }
        }
    }
}

// ---------------------------------------------------------------- lookup --
struct LevelIn {
    const float* p[kMaxLevels];
    int h[kMaxLevels];
    int w[kMaxLevels];
};

// Bilinear combination of an 8x8 window (rows = y offset, cols = x offset):
// channel a*7 + b (a the x offset, b the y offset); the four corner terms are
// added in the reference's loop order (i outer = x, j inner = y): (a,b),
// (a,b+1), (a+1,b), (a+1,b+1) (main.cu:1200-1216).
__device__ __forceinline__ void window_to_channels(const float (&win)[8][8], float dx, float dy,
                                                   float* o, int stride) {
    const float wx1 = dx, wx0 = 1.0f - dx, wy1 = dy, wy0 = 1.0f - dy;
#pragma unroll
    for (int a = 0; a < 7; a++) {
#pragma unroll
        for (int b = 0; b < 7; b++) {
            float s = win[b][a] * wx0 * wy0;
            s = s + win[b + 1][a] * wx0 * wy1;
            s = s + win[b][a + 1] * wx1 * wy0;
            s = s + win[b + 1][a + 1] * wx1 * wy1;
            o[(size_t)(a * 7 + b) * stride] = s;
        }
    }
}

// One thread per (source pixel, level, edge): zero-padded bilinear samples at
// (x0 - 3 + a, y0 - 3 + b), a,b in [0,7), from that pixel's own row of the
// level (main.cu:1175-1217). Non-finite coordinates give zeros.
__global__ __launch_bounds__(256) void k_corr_lookup(LevelIn lv, const float* __restrict__ coords,
                                                     float* __restrict__ out, int HW1,
                                                     int level_base, int nch) {
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    const int l = blockIdx.y;
    const int e = blockIdx.z;
    if (p >= HW1) return;
    const int H2 = lv.h[l], W2 = lv.w[l];
    const int lvl = level_base + l;
    const float cx = coords[(size_t)e * 2 * HW1 + p];
    const float cy = coords[(size_t)e * 2 * HW1 + HW1 + p];
    const float x0 = cx * (1.0f / (float)(1 << lvl));
    const float y0 = cy * (1.0f / (float)(1 << lvl));
    float* o = out + ((size_t)e * nch + (size_t)lvl * 49) * HW1 + p;
    if (!(isfinite(x0) && isfinite(y0))) {
#pragma unroll
        for (int k = 0; k < 49; k++) o[(size_t)k * HW1] = 0.0f;
        return;
    }
    const int ix = win_origin(cx, lvl), iy = win_origin(cy, lvl);
    const float* vol = lv.p[l] + ((size_t)e * HW1 + p) * (size_t)(H2 * W2);
    float win[8][8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int y = iy + j;
        const bool vy = (unsigned)y < (unsigned)H2;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int x = ix + i;
            const bool ok = vy && (unsigned)x < (unsigned)W2;
            win[j][i] = ok ? vol[y * W2 + x] : 0.0f;
        }
    }
    window_to_channels(win, x0 - floorf(x0), y0 - floorf(y0), o, HW1);
}

// Same lookup from the compact windows of the batched path: cells inside the
// level are read from the window buffer (contiguous 256 bytes per pixel and
// level), cells outside it are zero (they were never written).
__global__ __launch_bounds__(256) void k_corr_lookup_win(LevelIn lv, const float* __restrict__ wb,
                                                         const float* __restrict__ coords,
                                                         float* __restrict__ out, int HW1,
                                                         int nch) {
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    const int l = blockIdx.y;
    const int e = blockIdx.z;
    if (p >= HW1) return;
    const int H2 = lv.h[l], W2 = lv.w[l];
    const float cx = coords[(size_t)e * 2 * HW1 + p];
    const float cy = coords[(size_t)e * 2 * HW1 + HW1 + p];
    const float x0 = cx * (1.0f / (float)(1 << l));
    const float y0 = cy * (1.0f / (float)(1 << l));
    float* o = out + ((size_t)e * nch + (size_t)l * 49) * HW1 + p;
    if (!(isfinite(x0) && isfinite(y0))) {
#pragma unroll
        for (int k = 0; k < 49; k++) o[(size_t)k * HW1] = 0.0f;
        return;
    }
    const int ix = win_origin(cx, l), iy = win_origin(cy, l);
    // The window rows through a buffer resource over this edge and level: a
    // half row (4 cells, 16 bytes) with no cell in the grid, which the
    // correlation kernel never writes, is read at an offset past the range
    // and comes back as zeros without a memory access (22% of the pieces at
    // a +-8 pixel flow on 48 x 64 maps).
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(wb + win_index(e, l, 0, HW1, 0)), 0, kWinCells * HW1 * (int)sizeof(float),
        kBufWord3);
    const bool hx0 = ix + 3 >= 0 && ix < W2, hx1 = ix + 7 >= 0 && ix + 4 < W2;
    float win[8][8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const bool vy = (unsigned)(iy + j) < (unsigned)H2;
        const int off = (int)win_index(0, 0, j * 8, HW1, p) * (int)sizeof(float);
        // (whole-vector bit casts: this compiler's __builtin_bit_cast of a
        // subscripted vector element reads element 0 whatever the index)
        const float4 lo4 = __builtin_bit_cast(
            float4, __builtin_amdgcn_raw_buffer_load_b128(rs, vy && hx0 ? off : kBufDiscard, 0, 0));
        const float4 hi4 = __builtin_bit_cast(
            float4, __builtin_amdgcn_raw_buffer_load_b128(rs, vy && hx1 ? off + 16 : kBufDiscard, 0, 0));
        const float cell[8] = {lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const bool ok = vy && (unsigned)(ix + i) < (unsigned)W2;
            win[j][i] = ok ? cell[i] : 0.0f;
        }
    }
    window_to_channels(win, x0 - floorf(x0), y0 - floorf(y0), o, HW1);
}

template <typename Tin, bool WIN>
int launch_tile(slk_ctx* ctx, const Tin* fa, const Tin* fb, long fstride, const int* ia,
                const int* ib, const EdgeIdx& eidx, int n, float* const* lvl,
                const float* coords, float* win, int slot0, hipStream_t stream) {
    const int mtiles = (ctx->HW + kTileSrc - 1) / kTileSrc;
    const int nbands = (ctx->h + kBand - 1) / kBand;
    const int ncb = (ctx->w + kCols - 1) / kCols;
    const long total = (long)n * mtiles * nbands * ncb;
    if (total > 0x7fffffffL) return fail(SLK_E_ARG, "correlation grid too large");
    LevelOut lo{};
    if (lvl)
        for (int l = 0; l < kMaxLevels; l++) lo.p[l] = l < ctx->levels ? lvl[l] : nullptr;
    {
        ProfScope ps(ctx, WIN ? "corr_window" : "corr_pyramid", stream);
        constexpr bool f32 = std::is_same<Tin, float>::value;
        const bool split = (ctx->C % kKC == 0) && !(f32 && ctx->corr_prec == SLK_PREC_FP32);
        if (split) {
            constexpr int MODE = f32 ? kModeBF16x3 : kModeF16;
            hipLaunchKernelGGL((k_corr_mx<MODE, WIN>), dim3((unsigned)total), dim3(kWG), 0,
                               stream, fa, fb, fstride, ia, ib, eidx, lo, coords, win, slot0,
                               ctx->h, ctx->w, ctx->C, ctx->alpha, ctx->levels, mtiles, nbands,
                               ncb);
        } else {
            hipLaunchKernelGGL((k_corr_tile<Tin, WIN>), dim3((unsigned)total), dim3(kWG), 0,
                               stream, fa, fb, fstride, ia, ib, eidx, lo, coords, win, slot0,
                               ctx->h, ctx->w, ctx->C, ctx->alpha, ctx->levels, mtiles, nbands,
                               ncb);
        }
    }
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

int launch_lookup(slk_ctx* ctx, const LevelIn& lv, int nlev, int level_base, int nch,
                  const float* coords, float* out, int B, int HW1, hipStream_t stream) {
    if (B <= 0) return SLK_OK;
    dim3 grid((HW1 + 255) / 256, nlev, B);
    ProfScope ps(ctx, "corr_lookup", stream);
    hipLaunchKernelGGL(k_corr_lookup, grid, dim3(256), 0, stream, lv, coords, out, HW1, level_base,
                       nch);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

LevelIn level_in(slk_ctx* ctx, DevBuf* bufs) {
    LevelIn lv{};
    for (int l = 0; l < ctx->levels; l++) {
        lv.p[l] = bufs ? bufs[l].as<float>() : nullptr;
        lv.h[l] = ctx->lh[l];
        lv.w[l] = ctx->lw[l];
    }
    return lv;
}

int corr_batch_impl(slk_ctx* ctx, const void* fmaps, int dtype, long fstride, const int* ii_host,
                    const int* jj_host, const int* ii_dev, const int* jj_dev, int B,
                    const float* coords, float* out, hipStream_t stream) {
    if (!ctx || !fmaps || !coords || !out || B < 0)
        return fail(SLK_E_ARG, "corr_batch: null argument");
    if (dtype != SLK_F32 && dtype != SLK_F16) return fail(SLK_E_ARG, "corr_batch: bad dtype");
    if (fstride < (long)ctx->C * ctx->HW) return fail(SLK_E_ARG, "corr_batch: fmap_stride < C*h*w");
    const int HW = ctx->HW;
    const int nch = ctx->levels * 49;
    float* win = ctx->batch_win.as<float>();
    const LevelIn lv = level_in(ctx, nullptr);
    for (int b0 = 0; b0 < B; b0 += ctx->max_batch) {
        const int nb = B - b0 < ctx->max_batch ? B - b0 : ctx->max_batch;
        for (int s0 = 0; s0 < nb; s0 += kMaxEdgesPerLaunch) {
            const int n = nb - s0 < kMaxEdgesPerLaunch ? nb - s0 : kMaxEdgesPerLaunch;
            EdgeIdx eidx{};
            if (ii_host) {
                for (int k = 0; k < n; k++) {
                    eidx.ii[k] = ii_host[b0 + s0 + k];
                    eidx.jj[k] = jj_host[b0 + s0 + k];
                    if (eidx.ii[k] < 0 || eidx.jj[k] < 0)
                        return fail(SLK_E_ARG, "corr_batch: negative frame index");
                }
            }
            const int* ia = ii_host ? nullptr : ii_dev + b0 + s0;
            const int* ib = ii_host ? nullptr : jj_dev + b0 + s0;
            const float* cc = coords + (size_t)(b0 + s0) * 2 * HW;
            if (corr_split_supported(ctx) &&
                !(dtype == SLK_F32 && ctx->corr_prec == SLK_PREC_FP32)) {
                SLK_TRY(corr_split_windows(ctx, fmaps, dtype, fstride,
                                           ii_host ? eidx.ii : nullptr,
                                           ii_host ? eidx.jj : nullptr, ia, ib, n, cc, win, s0,
                                           stream));
            } else if (dtype == SLK_F32) {
                const float* f = static_cast<const float*>(fmaps);
                SLK_TRY((launch_tile<float, true>(ctx, f, f, fstride, ia, ib, eidx, n, nullptr, cc,
                                                  win, s0, stream)));
            } else {
                const _Float16* f = static_cast<const _Float16*>(fmaps);
                SLK_TRY((launch_tile<_Float16, true>(ctx, f, f, fstride, ia, ib, eidx, n, nullptr,
                                                     cc, win, s0, stream)));
            }
        }
        dim3 grid((HW + 255) / 256, ctx->levels, nb);
        ProfScope ps(ctx, "corr_lookup_win", stream);
        hipLaunchKernelGGL(k_corr_lookup_win, grid, dim3(256), 0, stream, lv, win,
                           coords + (size_t)b0 * 2 * HW, out + (size_t)b0 * nch * HW, HW, nch);
        SLK_HIP(hipGetLastError());
    }
    return SLK_OK;
}

}  // namespace

int corr_alloc(slk_ctx* ctx) {
    const size_t HW = (size_t)ctx->HW;
    SLK_TRY(ctx->batch_win.ensure((size_t)ctx->max_batch * HW * kMaxLevels * kWinCells *
                                  sizeof(float)));
    SLK_TRY(corr_split_alloc(ctx));
    for (int l = 0; l < ctx->levels; l++) {
        const size_t plane = (size_t)ctx->lh[l] * ctx->lw[l];
        SLK_TRY(ctx->single_lvl[l].ensure(HW * plane * sizeof(float)));
    }
    SLK_TRY(ctx->zero_idx.ensure(sizeof(int) * 4));
    SLK_HIP(hipMemset(ctx->zero_idx.ptr, 0, sizeof(int) * 4));
    // the zeroed buffers are in place before work on any stream (also a
    // non-blocking one) can read them
    SLK_HIP(hipDeviceSynchronize());
    return SLK_OK;
}

}  // namespace slk

using namespace slk;

extern "C" int slk_set_corr_precision(slk_ctx* ctx, int precision) {
    if (!ctx || (precision != SLK_PREC_BF16X3 && precision != SLK_PREC_FP32 &&
                 precision != SLK_PREC_F16X3))
        return fail(SLK_E_ARG, "set_corr_precision: bad argument");
    ctx->corr_prec = precision;
    return SLK_OK;
}

extern "C" int slk_corr_batch_build_and_sample(slk_ctx* ctx, const void* fmaps, int dtype,
                                               long fmap_stride, const int* ii_host,
                                               const int* jj_host, int B, const float* coords,
                                               float* out, hipStream_t stream) {
    if (B > 0 && (!ii_host || !jj_host)) return fail(SLK_E_ARG, "corr_batch: null indices");
    return corr_batch_impl(ctx, fmaps, dtype, fmap_stride, ii_host, jj_host, nullptr, nullptr, B,
                           coords, out, stream);
}

extern "C" int slk_corr_batch_build_and_sample_dev(slk_ctx* ctx, const void* fmaps, int dtype,
                                                   long fmap_stride, const int* ii_dev,
                                                   const int* jj_dev, int B,
                                                   const float* coords, float* out,
                                                   hipStream_t stream) {
    if (B > 0 && (!ii_dev || !jj_dev)) return fail(SLK_E_ARG, "corr_batch: null indices");
    return corr_batch_impl(ctx, fmaps, dtype, fmap_stride, nullptr, nullptr, ii_dev, jj_dev, B,
                           coords, out, stream);
}

extern "C" int slk_corr_prepare_frames(slk_ctx* ctx, const void* fmaps, int dtype,
                                       long fmap_stride, int nframes, hipStream_t stream) {
    if (!ctx || !fmaps) return fail(SLK_E_ARG, "corr_prepare_frames: null argument");
    if (dtype != SLK_F32 && dtype != SLK_F16)
        return fail(SLK_E_ARG, "corr_prepare_frames: bad dtype");
    if (fmap_stride < (long)ctx->C * ctx->HW)
        return fail(SLK_E_ARG, "corr_prepare_frames: fmap_stride < C*h*w");
    if (!corr_split_supported(ctx) || (dtype == SLK_F32 && ctx->corr_prec == SLK_PREC_FP32))
        return fail(SLK_E_ARG, "corr_prepare_frames: needs the split contraction (C % 16 == 0, "
                               "not SLK_PREC_FP32)");
    return corr_split_prepare(ctx, fmaps, dtype, fmap_stride, nframes, stream);
}

extern "C" int slk_corr_batch_build_and_sample_prepared(slk_ctx* ctx, const int* ii_host,
                                                        const int* jj_host, int B,
                                                        const float* coords, float* out,
                                                        hipStream_t stream) {
    if (!ctx || !coords || !out || B < 0 || (B > 0 && (!ii_host || !jj_host)))
        return fail(SLK_E_ARG, "corr_batch_prepared: null argument");
    if (ctx->prep_nframes <= 0)
        return fail(SLK_E_STATE, "corr_batch_prepared: no frames prepared");
    for (int e = 0; e < B; e++)
        if (ii_host[e] < 0 || jj_host[e] < 0 || ii_host[e] >= ctx->prep_nframes ||
            jj_host[e] >= ctx->prep_nframes)
            return fail(SLK_E_ARG, "corr_batch_prepared: frame index outside the prepared frames");
    const int HW = ctx->HW;
    const int nch = ctx->levels * 49;
    float* win = ctx->batch_win.as<float>();
    const LevelIn lv = level_in(ctx, nullptr);
    for (int b0 = 0; b0 < B; b0 += ctx->max_batch) {
        const int nb = B - b0 < ctx->max_batch ? B - b0 : ctx->max_batch;
        for (int s0 = 0; s0 < nb; s0 += kMaxEdgesPerLaunch) {
            const int n = nb - s0 < kMaxEdgesPerLaunch ? nb - s0 : kMaxEdgesPerLaunch;
            SLK_TRY(corr_split_windows_prepared(ctx, ii_host + b0 + s0, jj_host + b0 + s0, n,
                                                coords + (size_t)(b0 + s0) * 2 * HW, win, s0,
                                                stream));
        }
        dim3 grid((HW + 255) / 256, ctx->levels, nb);
        ProfScope ps(ctx, "corr_lookup_win", stream);
        hipLaunchKernelGGL(k_corr_lookup_win, grid, dim3(256), 0, stream, lv, win,
                           coords + (size_t)b0 * 2 * HW, out + (size_t)b0 * nch * HW, HW, nch);
        SLK_HIP(hipGetLastError());
    }
    return SLK_OK;
}

extern "C" int slk_corr_build(slk_ctx* ctx, const void* f_i, const void* f_j, int dtype,
                              hipStream_t stream) {
    if (!ctx || !f_i || !f_j) return fail(SLK_E_ARG, "corr_build: null argument");
    float* lvl[kMaxLevels];
    for (int l = 0; l < ctx->levels; l++) lvl[l] = ctx->single_lvl[l].as<float>();
    const int* z = ctx->zero_idx.as<int>();
    EdgeIdx eidx{};
    if (dtype == SLK_F32) {
        SLK_TRY((launch_tile<float, false>(ctx, static_cast<const float*>(f_i),
                                           static_cast<const float*>(f_j), 0, z, z, eidx, 1, lvl,
                                           nullptr, nullptr, 0, stream)));
    } else if (dtype == SLK_F16) {
        SLK_TRY((launch_tile<_Float16, false>(ctx, static_cast<const _Float16*>(f_i),
                                              static_cast<const _Float16*>(f_j), 0, z, z, eidx, 1,
                                              lvl, nullptr, nullptr, 0, stream)));
    } else {
        return fail(SLK_E_ARG, "corr_build: bad dtype");
    }
    ctx->single_built = true;
    return SLK_OK;
}

extern "C" int slk_corr_sample(slk_ctx* ctx, const float* coords, float* out, hipStream_t stream) {
    if (!ctx || !coords || !out) return fail(SLK_E_ARG, "corr_sample: null argument");
    if (!ctx->single_built) return fail(SLK_E_STATE, "corr_sample: no volume built");
    const LevelIn lv = level_in(ctx, ctx->single_lvl);
    return launch_lookup(ctx, lv, ctx->levels, 0, ctx->levels * 49, coords, out, 1, ctx->HW,
                         stream);
}

extern "C" int slk_corr_level(slk_ctx* ctx, int level, const float** ptr, int* h2, int* w2) {
    if (!ctx || level < 0 || level >= ctx->levels) return fail(SLK_E_ARG, "corr_level: bad level");
    if (ptr) *ptr = ctx->single_lvl[level].as<float>();
    if (h2) *h2 = ctx->lh[level];
    if (w2) *w2 = ctx->lw[level];
    return SLK_OK;
}

namespace {
__global__ void k_avg_pool_2x2(const float* __restrict__ in, float* __restrict__ out, long N, int H,
                               int W) {
    const int oH = H / 2, oW = W / 2;
    const long total = N * oH * oW;
    for (long idx = blockIdx.x * (long)blockDim.x + threadIdx.x; idx < total;
         idx += (long)gridDim.x * blockDim.x) {
        const long n = idx / (oH * oW);
        const int rem = (int)(idx - n * oH * oW);
        const int oy = rem / oW, ox = rem % oW;
        const float* src = in + (size_t)n * H * W + (2 * oy) * W + 2 * ox;
        float s = src[0] + src[1];
        s = s + src[W];
        s = s + src[W + 1];
        out[idx] = 0.25f * s;
    }
}

__global__ void k_coords_hw2_to_2hw(const float* __restrict__ hw2, float* __restrict__ chw, int M,
                                    int HW) {
    const long idx = blockIdx.x * (long)blockDim.x + threadIdx.x;
    if (idx >= (long)M * HW) return;
    const long e = idx / HW, k = idx % HW;
    chw[e * 2 * HW + k] = hw2[idx * 2 + 0];
    chw[e * 2 * HW + HW + k] = hw2[idx * 2 + 1];
}
}  // namespace

extern "C" int slk_avg_pool_2x2(const float* in, float* out, long N, int H, int W,
                                hipStream_t stream) {
    if (!in || !out || N < 0 || H < 0 || W < 0) return fail(SLK_E_ARG, "avg_pool_2x2: bad args");
    const long total = N * (H / 2) * (W / 2);
    if (total == 0) return SLK_OK;
    long blocks = (total + 255) / 256;
    if (blocks > 65536 * 4) blocks = 65536 * 4;
    hipLaunchKernelGGL(k_avg_pool_2x2, dim3((unsigned)blocks), dim3(256), 0, stream, in, out, N, H,
                       W);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

extern "C" int slk_corr_sample_level(const float* volumes, const float* coords, float* corr_out,
                                     int M, int r, int H1, int W1, int H2, int W2, int hw,
                                     float coord_scale, int level_idx, hipStream_t stream) {
    if (r != 3) return fail(SLK_E_ARG, "corr_sample_level: only r = 3");
    if (!volumes || !coords || !corr_out || M < 0 || H1 * W1 != hw || level_idx < 0 ||
        level_idx >= kMaxLevels)
        return fail(SLK_E_ARG, "corr_sample_level: bad args");
    if (coord_scale != 1.0f / (float)(1 << level_idx))
        return fail(SLK_E_ARG, "corr_sample_level: coord_scale must be 2^-level_idx");
    LevelIn lv{};
    lv.p[0] = volumes;
    lv.h[0] = H2;
    lv.w[0] = W2;
    // channels [level_idx*49, +49) of a [M][196][hw] buffer, like the reference
    return launch_lookup(nullptr, lv, 1, level_idx, 196, coords, corr_out, M, hw, stream);
}

extern "C" int slk_coords_hw2_to_2hw(const float* hw2, float* chw, int M, int HW,
                                     hipStream_t stream) {
    if (!hw2 || !chw || M < 0 || HW < 0) return fail(SLK_E_ARG, "coords_hw2_to_2hw: bad args");
    const long total = (long)M * HW;
    if (total == 0) return SLK_OK;
    hipLaunchKernelGGL(k_coords_hw2_to_2hw, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       stream, hw2, chw, M, HW);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

// ------------------------------------------------ no-allocation batched path
// slk_corr_batch_build_and_sample_dev_noalloc runs the batched path with its
// scratch (feature slots, tile lists and counters, lookup windows) carved
// from one file-scope device array instead of a context's buffers. The array
// is a host-side stand-in in host code: its device address on the current
// device comes from hipGetSymbolAddress, taken once per device on the first
// call there, and only that address is handed to kernels.
namespace {
constexpr size_t kNoAllocBytes = size_t(64) << 20;
constexpr int kNoAllocDevices = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

namespace {
std::mutex g_noalloc_mu;
unsigned char* g_noalloc_ptr[kNoAllocDevices];
int g_noalloc_cus[kNoAllocDevices];

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// Device address of `scratch` and the CU count of the current device.
int noalloc_scratch(unsigned char** ptr, int* cus, int* device) {
    int dev = 0;
    SLK_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kNoAllocDevices)
        return fail(SLK_E_ARG, "corr_noalloc: device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
        void* p = nullptr;
        SLK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        int n = 0;
        SLK_HIP(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
        g_noalloc_cus[dev] = n;
        g_noalloc_ptr[dev] = static_cast<unsigned char*>(p);
    }
    *ptr = g_noalloc_ptr[dev];
    *cus = g_noalloc_cus[dev];
    *device = dev;
    return SLK_OK;
}
}  // namespace

extern "C" int slk_corr_batch_build_and_sample_dev_noalloc(
    const void* fmaps, int dtype, long fmap_stride, const int* ii_dev, const int* jj_dev, int B,
    const float* coords, float* out, int h, int w, int C, float corr_scale,
    hipStream_t stream) {
    if (B < 0 || (B > 0 && (!ii_dev || !jj_dev)))
        return fail(SLK_E_ARG, "corr_noalloc: null indices or B < 0");
    if (h < 8 || w < 8 || h > 65536 || w > 65536 || (long)h * w >= (1L << 21))
        return fail(SLK_E_ARG, "corr_noalloc: need 8 <= h, w <= 2^16 and h*w < 2^21");
    if (C < 16 || C % 16 != 0)
        return fail(SLK_E_ARG, "corr_noalloc: C must be a positive multiple of 16");
    if (dtype != SLK_F32 && dtype != SLK_F16) return fail(SLK_E_ARG, "corr_noalloc: bad dtype");
    slk_ctx c;  // a stack context over the static scratch: nothing here allocates
    c.h = h;
    c.w = w;
    c.HW = h * w;
    c.C = C;
    c.levels = kMaxLevels;
    c.radius = 3;
    c.alpha = corr_scale;
    c.corr_prec = SLK_PREC_F16X3;
    for (int l = 0; l < kMaxLevels; l++) {
        c.lh[l] = h >> l;
        c.lw[l] = w >> l;
    }
    size_t slot = 0, tiles = 0, order = 0, ctr = 0;
    corr_split_footprint(&c, &slot, &tiles, &order, &ctr);
    const size_t win = (size_t)c.HW * kMaxLevels * kWinCells * sizeof(float);
    const size_t per_edge = 2 * align256(slot) + align256(tiles) + align256(order) +
                            align256(win);
    const size_t fixed = align256(ctr);
    const size_t fit = per_edge + fixed <= kNoAllocBytes ? (kNoAllocBytes - fixed) / per_edge : 0;
    if (fit < 1)
        return fail(SLK_E_ARG, "corr_noalloc: one edge of this map size needs more than the "
                               "64 MiB static scratch");
    if (B == 0) return SLK_OK;
    unsigned char* base = nullptr;
    int cus = 0, dev = 0;
    SLK_TRY(noalloc_scratch(&base, &cus, &dev));
    c.device = dev;
    const int n = (int)std::min<size_t>(fit, kMaxEdgesPerLaunch);
    c.max_batch = n;
    size_t at = 0;
    auto carve = [&](DevBuf& b, size_t bytes) {
        b.ptr = base + at;
        b.bytes = bytes;
        at += align256(bytes);
    };
    carve(c.split_feat, 2 * (size_t)n * align256(slot));
    carve(c.tile_list, (size_t)n * tiles);
    carve(c.src_order, (size_t)n * order);
    carve(c.tile_ctr, ctr);
    carve(c.batch_win, (size_t)n * win);
    if (at > kNoAllocBytes) return fail(SLK_E_ARG, "corr_noalloc: scratch layout overflow");
    c.ws_grid = corr_split_grid(cus);
    return corr_batch_impl(&c, fmaps, dtype, fmap_stride, nullptr, nullptr, ii_dev, jj_dev, B,
                           coords, out, stream);
}
