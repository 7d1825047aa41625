// Stage 4 of the Engram lookup path on gfx950, the training side: touched-row dedup with
// coalesced gradient sums, the global gradient norm for clipping, and the lazy / row-wise Adam
// update of the touched rows with stochastic rounding to bf16.
//
// Reference:
//   dedup      micro_engram/rows.py:81 (torch.unique(return_inverse)), 117-118 and 144-146
//              (zeros().index_add_(0, inv, g)): unique keys ascending, the inverse index, and the
//              fp32 sum of each key's gradient rows in the order the rows appear
//   sumsq      rows.py:214-220 (the squared norm RowTables.clip scales against)
//   clip       rows.py:221-231 (the gradients scaled in place by min(max_norm / (norm + 1e-6), 1))
//   adam       micro_engram/optim.py:65-133, the sparse-gradient branch (88-97), per-row second
//              moment (112-114) and write-back with stochastic_bf16 (33-44, 120-132)
//
// Dedup, in two halves: the keys (sorted unique keys, the inverse, and a segment plan: every
// position in sorted key order, each unique key's first index and first position) depend
// only on the row ids, and the sums read the gradients through the plan. Two key paths with the
// same results. Keys whose bits below a group fit 32 (the usual case: table offset + row): three
// launches -- per-tile grouping by the high key bits, one workgroup per group that sorts the
// group's (low key bits, position) composites in LDS and counts its unique keys, and one that
// numbers them after the earlier groups' and writes the unique keys, the inverse and the plan
// (gd_* kernels below). Wider keys: a stable LSD radix sort of (key, position) pairs, 8 key bits
// per pass (per-block digit histograms, then a scatter that ranks equal digits inside each wave
// with 8 ballots, lower lane = earlier element), and segment heads. The sums: one thread per
// (segment, 4 columns), a segment's gradient rows added in ascending position order starting
// from +0.0 -- the order, and so the rounding, of CPU index_add_.
#include "me_common.h"

#include <algorithm>
#include <cmath>

namespace me {
namespace {

constexpr int kThreads = 256;
constexpr int kItems = 8;                        // elements per thread per tile
constexpr int kTile = kThreads * kItems;         // 2048 elements per sort block
constexpr int kBins = 256;                       // 8-bit digits

__device__ __forceinline__ uint64_t lanes_below(int lane) { return (1ull << lane) - 1ull; }

// ---- radix sort -----------------------------------------------------------------------------
// hist[digit * stride + tile]: row `digit` holds that digit's count in every tile; rows are
// padded to a multiple of 4 tiles (zeros) so a row reads as 16-byte words.
__global__ __launch_bounds__(kThreads) void rs_hist(const uint64_t *keys, int64_t n, int shift,
                                                    uint32_t *hist, int nblocks, int stride) {
    __shared__ uint32_t s[kBins];
    const int tid = threadIdx.x;
    s[tid] = 0;
    __syncthreads();
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const int64_t idx = base + i * kThreads + tid;
        if (idx < n) atomicAdd(&s[(keys[idx] >> shift) & (kBins - 1)], 1u);
    }
    __syncthreads();
    hist[static_cast<int64_t>(tid) * stride + blockIdx.x] = s[tid];
    if (blockIdx.x == 0)
        for (int b = nblocks; b < stride; ++b) hist[static_cast<int64_t>(tid) * stride + b] = 0u;
}

// Exclusive prefix sum of v[0..total) in place, one workgroup. If total_out is given, the sum
// of all entries is written there too.
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t x, int lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    return x;
}

// Scatter of one tile. Its output base for digit d = (all keys with a smaller digit) + (keys
// with digit d in earlier tiles): thread d reads row d of the histogram as 16-byte words,
// summing the earlier tiles and all tiles, and a scan of the 256 totals across the workgroup
// orders the digits. Every tile derives its bases itself, so a pass is two launches.
__global__ __launch_bounds__(kThreads) void rs_scatter(const uint64_t *keys_in, const uint32_t *pos_in,
                                                       uint64_t *keys_out, uint32_t *pos_out,
                                                       int64_t n, int shift, const uint32_t *hist,
                                                       int stride) {
    __shared__ uint32_t s_base[kBins];
    __shared__ uint32_t s_wcnt[kThreads / 64][kBins];
    __shared__ uint32_t s_wtot[kThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    {
        static_assert(kThreads == kBins, "one thread per digit");
        const uint4 *row = reinterpret_cast<const uint4 *>(hist + static_cast<int64_t>(tid) * stride);
        const int words = stride / 4, me = static_cast<int>(blockIdx.x);
        uint32_t mine = 0, tot = 0;
        for (int q0 = 0; q0 < words; q0 += 8) {
            uint4 x[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) x[u] = q0 + u < words ? row[q0 + u] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int t0 = (q0 + u) * 4;
                const uint32_t c[4] = {x[u].x, x[u].y, x[u].z, x[u].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    tot += c[e];
                    if (t0 + e < me) mine += c[e];
                }
            }
        }
        const uint32_t incl = wave_inclusive_scan(tot, lane);
        if (lane == 63) s_wtot[wave] = incl;
        __syncthreads();
        uint32_t before = 0;
        for (int w = 0; w < wave; ++w) before += s_wtot[w];
        s_base[tid] = before + incl - tot + mine;
    }
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
    for (int i = 0; i < kItems; ++i) {
        const int64_t idx = base + i * kThreads + tid;
        const bool valid = idx < n;
        const uint64_t key = valid ? keys_in[idx] : 0ull;
        const uint32_t pos = valid ? (pos_in != nullptr ? pos_in[idx] : static_cast<uint32_t>(idx)) : 0u;
        const int digit = static_cast<int>((key >> shift) & (kBins - 1));
#pragma unroll
        for (int q = 0; q < kBins / 64; ++q) s_wcnt[wave][lane * (kBins / 64) + q] = 0u;
        // lanes of this wave holding the same digit
        uint64_t same = __ballot(valid);
#pragma unroll
        for (int bit = 0; bit < 8; ++bit) {
            const bool set = (digit >> bit) & 1;
            const uint64_t b = __ballot(set);
            same &= set ? b : ~b;
        }
        const int rank = __popcll(same & lanes_below(lane));
        __syncthreads();  // counts cleared (and the previous chunk's base update is done)
        if (valid && rank == 0) s_wcnt[wave][digit] = static_cast<uint32_t>(__popcll(same));
        __syncthreads();
        if (valid) {
            uint32_t off = s_base[digit] + static_cast<uint32_t>(rank);
            for (int w = 0; w < wave; ++w) off += s_wcnt[w][digit];
            keys_out[off] = key;
            pos_out[off] = pos;
        }
        __syncthreads();
        uint32_t add = 0;
#pragma unroll
        for (int w = 0; w < kThreads / 64; ++w) add += s_wcnt[w][tid];
        s_base[tid] += add;
        __syncthreads();  // the next chunk clears s_wcnt and reads s_base
    }
}

// ---- segments of the sorted keys -------------------------------------------------------------
// Both dedup paths leave a segment plan the sums read: spos (every position, in sorted key
// order), seg_start (each unique key's first index into spos, then n) and seg_pos (each unique
// key's first position, so the sums start its first row without going through spos).
// Tile layout for the segment pass: thread t owns elements [t * kItems, (t + 1) * kItems) of
// its block's tile, so a block-level exclusive scan of per-thread head counts numbers the heads.
__device__ __forceinline__ bool is_head(const uint64_t *k, int64_t i) {
    return i == 0 || k[i] != k[i - 1];
}

__global__ __launch_bounds__(kThreads) void seg_count(const uint64_t *skeys, int64_t n,
                                                      uint32_t *block_heads) {
    __shared__ uint32_t s[kThreads];
    const int tid = threadIdx.x;
    const int64_t b = static_cast<int64_t>(blockIdx.x) * kTile + static_cast<int64_t>(tid) * kItems;
    uint32_t c = 0;
    for (int i = 0; i < kItems; ++i)
        if (b + i < n && is_head(skeys, b + i)) ++c;
    s[tid] = c;
    __syncthreads();
    for (int off = kThreads / 2; off > 0; off >>= 1) {
        if (tid < off) s[tid] += s[tid + off];
        __syncthreads();
    }
    if (tid == 0) block_heads[blockIdx.x] = s[0];
}

__global__ __launch_bounds__(kThreads) void seg_write(const uint64_t *skeys, const uint32_t *spos,
                                                      int64_t n, const uint32_t *block_heads,
                                                      int nblocks, int64_t *uniq, int64_t *inv,
                                                      uint32_t *seg_start, uint32_t *seg_pos,
                                                      int64_t *count) {
    __shared__ uint32_t s[kThreads];
    __shared__ uint32_t s_before[kThreads / 64], s_all[kThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    {   // heads in the tiles before this one (and in all tiles, for the count)
        uint32_t before = 0, all = 0;
        for (int b = tid; b < nblocks; b += kThreads) {
            const uint32_t c = block_heads[b];
            all += c;
            if (b < static_cast<int>(blockIdx.x)) before += c;
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            before += __shfl_xor(before, off, 64);
            all += __shfl_xor(all, off, 64);
        }
        if (lane == 0) {
            s_before[wave] = before;
            s_all[wave] = all;
        }
    }
    const int64_t b = static_cast<int64_t>(blockIdx.x) * kTile + static_cast<int64_t>(tid) * kItems;
    uint32_t c = 0;
    for (int i = 0; i < kItems; ++i)
        if (b + i < n && is_head(skeys, b + i)) ++c;
    s[tid] = c;
    __syncthreads();
    for (int off = 1; off < kThreads; off <<= 1) {
        const uint32_t t = tid >= off ? s[tid - off] : 0u;
        __syncthreads();
        s[tid] += t;
        __syncthreads();
    }
    uint32_t tile_base = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) {
        tile_base += s_before[w];
        total += s_all[w];
    }
    if (blockIdx.x == 0 && tid == 0) *count = total;
    // heads before this thread's first element, over the whole array
    uint32_t heads = tile_base + s[tid] - c;
    for (int i = 0; i < kItems; ++i) {
        const int64_t idx = b + i;
        if (idx >= n) break;
        const uint32_t pos = spos[idx];
        if (is_head(skeys, idx)) {
            uniq[heads] = static_cast<int64_t>(skeys[idx]);
            seg_start[heads] = static_cast<uint32_t>(idx);
            seg_pos[heads] = pos;
            ++heads;
        }
        inv[pos] = static_cast<int64_t>(heads) - 1;
        if (idx == n - 1) seg_start[heads] = static_cast<uint32_t>(n);
    }
}

__global__ void write_zero_count(int64_t *count) { *count = 0; }

// ---- segment sums ----------------------------------------------------------------------------
// Each unique key's gradient rows summed in sorted (= position) order, starting from +0.0 like
// zeros().index_add_(). A thread owns one run of kCols columns of one segment: the segment's
// bounds and first position are independent loads, and rows after the first are fetched
// kSumBatch at a time (all positions, then all rows in flight) and added in order.
__device__ __forceinline__ void load_cols(const float *p, float (&x)[4]) {
    const float4 v = *reinterpret_cast<const float4 *>(p);
    x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
}
__device__ __forceinline__ void load_cols(const uint16_t *p, float (&x)[4]) {
    const uint2 v = *reinterpret_cast<const uint2 *>(p);
    x[0] = bf16_bits_to_float(static_cast<uint16_t>(v.x));
    x[1] = bf16_bits_to_float(static_cast<uint16_t>(v.x >> 16));
    x[2] = bf16_bits_to_float(static_cast<uint16_t>(v.y));
    x[3] = bf16_bits_to_float(static_cast<uint16_t>(v.y >> 16));
}
__device__ __forceinline__ void load_cols(const float *p, float (&x)[1]) { x[0] = *p; }
__device__ __forceinline__ void load_cols(const uint16_t *p, float (&x)[1]) {
    x[0] = bf16_bits_to_float(*p);
}

// Rows of a segment past its first, loaded per step (positions, then rows, all in flight): the
// longest segment (a hot key's repeats) is the kernel's critical path.
constexpr int kSumBatch = 16;

template <typename G, int kCols>
__global__ __launch_bounds__(kThreads) void seg_sum(const G *grads, uint32_t dim, const uint32_t *spos,
                                                    const uint32_t *seg_start, const uint32_t *seg_pos,
                                                    const int64_t *count, uint32_t max_segs, float *gsum) {
    const uint32_t runs = dim / kCols;
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    const uint32_t seg = t / runs;
    if (seg >= max_segs) return;
    const uint32_t c0 = (t - seg * runs) * kCols;
    const uint32_t lo = seg_start[seg], hi = seg_start[seg + 1], first = seg_pos[seg];
    if (static_cast<int64_t>(seg) >= *count) return;
    float acc[kCols], x[kCols];
    load_cols(grads + static_cast<uint64_t>(first) * dim + c0, x);
#pragma unroll
    for (int c = 0; c < kCols; ++c) acc[c] = 0.f + x[c];
    for (uint32_t i = lo + 1; i < hi; i += kSumBatch) {
        const uint32_t m = hi - i < static_cast<uint32_t>(kSumBatch) ? hi - i : kSumBatch;
        uint32_t q[kSumBatch];
        float y[kSumBatch][kCols];
#pragma unroll
        for (int v = 0; v < kSumBatch; ++v) q[v] = static_cast<uint32_t>(v) < m ? spos[i + v] : first;
#pragma unroll
        for (int v = 0; v < kSumBatch; ++v) load_cols(grads + static_cast<uint64_t>(q[v]) * dim + c0, y[v]);
#pragma unroll
        for (int v = 0; v < kSumBatch; ++v)
            if (static_cast<uint32_t>(v) < m)
#pragma unroll
                for (int c = 0; c < kCols; ++c) acc[c] = acc[c] + y[v][c];
    }
    float *out = gsum + static_cast<uint64_t>(seg) * dim + c0;
    if constexpr (kCols == 4)
        *reinterpret_cast<float4 *>(out) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    else
        out[0] = acc[0];
}

// ---- group dedup ------------------------------------------------------------------------------
// The dedup when the key bits below a group fit 32: a key's group is its high bits (key >>
// shift, a few hundred keys per group on average), and the composites (low key bits << 32 |
// position) of one group are distinct, so their order is the stable order of the keys. Three
// launches, no device-scope atomics:
//   gd_tile   per tile of 2048 keys: an LDS histogram over the groups, its exclusive prefix
//             (the tile's offset of every group, written as a row of `off`), and the tile's
//             composites grouped by group into its slice of tile_comp;
//   gd_group  per group: its runs from every tile gathered into LDS, bucketed by the top 8 low
//             key bits, each composite ranked inside its bucket (the rest of a bucket is a few
//             composites, or the repeats of one hot key), written sorted into comp at the
//             group's start (the sum of its offsets over the tiles), its unique keys counted;
//   gd_emit   per group: its unique keys numbered after the earlier groups' (a block sum of
//             their counts), then uniq, inv and the segment plan.
// A group larger than LDS is sorted by its workgroup in global memory (stable LSD radix sort).
constexpr int kGdTile = kTile;            // keys per gd_tile workgroup
constexpr uint32_t kGdMaxGroups = 1024;   // groups (LDS counters of gd_tile)
constexpr uint32_t kGdMaxTiles = 1024;    // tiles (n up to 2^21)
constexpr int kGdCap = 2048;              // composites a group may sort in LDS
constexpr int64_t kGdMean = 256;          // keys per group aimed at (at most twice that)
constexpr int kGdSubBits = 10;            // a group's LDS sort: buckets of its top low key bits
constexpr int kGdSub = 1 << kGdSubBits;

// Group of a key; keys outside [0, key_bound) (outside the contract) land in the last group
// instead of outside the arrays.
__device__ __forceinline__ uint32_t group_of(uint64_t key, int shift, uint32_t ng) {
    const uint64_t g = key >> shift;
    return g < ng ? static_cast<uint32_t>(g) : ng - 1;
}

__device__ __forceinline__ uint64_t composite(uint64_t key, uint32_t g, int shift, uint32_t pos) {
    return ((key - (static_cast<uint64_t>(g) << shift)) << 32) | pos;
}

// Exclusive scan of the 256 per-thread values v across the workgroup; *total gets the sum.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t *s_wtot, uint32_t *total) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t incl = wave_inclusive_scan(v, lane);
    if (lane == 63) s_wtot[wave] = incl;
    __syncthreads();
    uint32_t before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) {
        const uint32_t x = s_wtot[w];
        before += w < wave ? x : 0u;
        all += x;
    }
    __syncthreads();  // s_wtot may be reused
    *total = all;
    return before + incl - v;
}

// Tile t: counts per group, their exclusive prefix as row t of off ([tiles][ng + 1]), and the
// tile's composites at tile_comp[t * kGdTile + prefix + slot] (slots by LDS counters).
__global__ __launch_bounds__(kThreads) void gd_tile(const uint64_t *keys, int64_t n, int shift, uint32_t ng,
                                                    uint64_t *tile_comp, uint32_t *off) {
    __shared__ uint32_t s_cnt[kGdMaxGroups + 1];
    __shared__ uint32_t s_wtot[kThreads / 64];
    const int tid = threadIdx.x;
    for (uint32_t g = tid; g <= ng; g += kThreads) s_cnt[g] = 0u;
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kGdTile;
    uint64_t k[kItems];
#pragma unroll
    for (int e = 0; e < kItems; ++e) {
        const int64_t i = base + e * kThreads + tid;
        k[e] = i < n ? keys[i] : 0ull;
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < kItems; ++e)
        if (base + e * kThreads + tid < n) atomicAdd(&s_cnt[group_of(k[e], shift, ng)], 1u);
    __syncthreads();
    // exclusive prefix over the groups: thread tid owns groups [tid * per, tid * per + per)
    const uint32_t per = (ng + kThreads - 1) / kThreads;
    const uint32_t g0 = static_cast<uint32_t>(tid) * per;
    uint32_t mine = 0;
    for (uint32_t q = 0; q < per; ++q)
        if (g0 + q < ng) mine += s_cnt[g0 + q];
    uint32_t total;
    uint32_t run = block_exclusive_scan(mine, s_wtot, &total);
    for (uint32_t q = 0; q < per; ++q)
        if (g0 + q < ng) {
            const uint32_t c = s_cnt[g0 + q];
            s_cnt[g0 + q] = run;
            run += c;
        }
    if (tid == 0) s_cnt[ng] = total;
    __syncthreads();
    uint32_t *row = off + static_cast<uint64_t>(blockIdx.x) * (ng + 1);
    for (uint32_t g = tid; g <= ng; g += kThreads) row[g] = s_cnt[g];
    __syncthreads();  // the row is read before the counters move on
    uint64_t *out = tile_comp + base;
#pragma unroll
    for (int e = 0; e < kItems; ++e) {
        const int64_t i = base + e * kThreads + tid;
        if (i < n) {
            const uint32_t g = group_of(k[e], shift, ng);
            const uint32_t slot = atomicAdd(&s_cnt[g], 1u);
            out[slot] = composite(k[e], g, shift, static_cast<uint32_t>(i));
        }
    }
}

// Stable LSD radix sort of the n composites at a (ping-ponging with t, 8-bit digits, `bits`
// significant bits) by one workgroup; the result ends in a.
__device__ void wg_radix_sort(uint64_t *a, uint64_t *t, uint32_t n, int bits) {
    __shared__ uint32_t s_hist[kBins];
    __shared__ uint32_t s_wcnt[kThreads / 64][kBins];
    __shared__ uint32_t s_wtot[kThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int passes = (bits + 7) / 8;
    uint64_t *src = a, *dst = t;
    for (int pass = 0; pass < passes; ++pass) {
        const int sh = 8 * pass;
        s_hist[tid] = 0u;
        __syncthreads();
        for (uint32_t i = tid; i < n; i += kThreads) atomicAdd(&s_hist[(src[i] >> sh) & (kBins - 1)], 1u);
        __syncthreads();
        {   // exclusive scan of the 256 digit counts, thread d holds digit d
            const uint32_t c = s_hist[tid];
            const uint32_t incl = wave_inclusive_scan(c, lane);
            if (lane == 63) s_wtot[wave] = incl;
            __syncthreads();
            uint32_t before = 0;
            for (int w = 0; w < wave; ++w) before += s_wtot[w];
            s_hist[tid] = before + incl - c;  // the digit's next output slot
        }
        __syncthreads();
        for (uint32_t i0 = 0; i0 < n; i0 += kThreads) {
            const uint32_t i = i0 + tid;
            const bool valid = i < n;
            const uint64_t v = valid ? src[i] : 0ull;
            const int digit = static_cast<int>((v >> sh) & (kBins - 1));
#pragma unroll
            for (int u = 0; u < kBins / 64; ++u) s_wcnt[wave][lane * (kBins / 64) + u] = 0u;
            uint64_t same = __ballot(valid);
#pragma unroll
            for (int bit = 0; bit < 8; ++bit) {
                const bool set = (digit >> bit) & 1;
                const uint64_t bb = __ballot(set);
                same &= set ? bb : ~bb;
            }
            const int rank = __popcll(same & lanes_below(lane));
            __syncthreads();
            if (valid && rank == 0) s_wcnt[wave][digit] = static_cast<uint32_t>(__popcll(same));
            __syncthreads();
            if (valid) {
                uint32_t o = s_hist[digit] + static_cast<uint32_t>(rank);
                for (int w = 0; w < wave; ++w) o += s_wcnt[w][digit];
                dst[o] = v;
            }
            __syncthreads();
            uint32_t add = 0;
#pragma unroll
            for (int w = 0; w < kThreads / 64; ++w) add += s_wcnt[w][tid];
            s_hist[tid] += add;
            __syncthreads();
        }
        uint64_t *x = src;
        src = dst;
        dst = x;
    }
    if (src != a)
        for (uint32_t i = tid; i < n; i += kThreads) a[i] = src[i];
    __syncthreads();
}

// Group g: its composites sorted into comp[gstart[g], gstart[g] + size) and its unique key
// count into ucount[g]. The runs: tile t holds the group's composites at off[t][g] ..
// off[t][g + 1] of its slice; the group starts at the sum of off[t][g] over the tiles (every
// key of an earlier group, in every tile).
__global__ __launch_bounds__(kThreads) void gd_group(const uint64_t *tile_comp, const uint32_t *off,
                                                     uint32_t ntiles, uint32_t ng, int shift, int64_t n,
                                                     uint64_t *comp, uint64_t *tmp, uint32_t *gstart,
                                                     uint32_t *ucount) {
    __shared__ uint64_t s_a[kGdCap];
    __shared__ uint64_t s_b[kGdCap];
    __shared__ uint16_t s_map[kGdCap];           // run (tile) of each of the group's composites
    __shared__ uint32_t s_run[kGdMaxTiles + 1];  // run t lands at [s_run[t], s_run[t + 1])
    __shared__ uint32_t s_src[kGdMaxTiles];      // run t's first index into tile_comp
    __shared__ uint32_t s_sb[kGdSub + 1];        // bucket starts
    __shared__ uint32_t s_cur[kGdSub];           // bucket fill counters
    __shared__ uint32_t s_wtot[kThreads / 64];
    __shared__ uint32_t s_red[kThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t g = blockIdx.x;
    // ---- the runs: thread tid owns tiles [tid * per, tid * per + per)
    const uint32_t per = (ntiles + kThreads - 1) / kThreads;
    const uint32_t t0 = static_cast<uint32_t>(tid) * per;
    uint32_t lo[4], len[4];  // per <= 4 (ntiles <= 1024)
    uint32_t mine = 0, before_sum = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        lo[q] = 0u;
        len[q] = 0u;
        if (static_cast<uint32_t>(q) < per && t0 + q < ntiles) {
            const uint32_t *row = off + static_cast<uint64_t>(t0 + q) * (ng + 1);
            lo[q] = row[g];
            len[q] = row[g + 1] - lo[q];
            mine += len[q];
            before_sum += lo[q];
        }
    }
    uint32_t size, gs;
    uint32_t run = block_exclusive_scan(mine, s_wtot, &size);
    block_exclusive_scan(before_sum, s_wtot, &gs);
    const bool in_lds = size <= static_cast<uint32_t>(kGdCap);
#pragma unroll
    for (int q = 0; q < 4; ++q)
        if (static_cast<uint32_t>(q) < per && t0 + q < ntiles) {
            s_run[t0 + q] = run;
            s_src[t0 + q] = (t0 + q) * static_cast<uint32_t>(kGdTile) + lo[q];
            if (in_lds)
                for (uint32_t j = 0; j < len[q]; ++j) s_map[run + j] = static_cast<uint16_t>(t0 + q);
            run += len[q];
        }
    if (tid == 0) {
        s_run[ntiles] = size;
        gstart[g] = gs;
        if (g == ng - 1) gstart[ng] = static_cast<uint32_t>(n);
    }
    __syncthreads();
    // composite k of the group: k - s_run[t] into run t
    auto src_of = [&](uint32_t k, uint32_t t) { return s_src[t] + (k - s_run[t]); };
    uint32_t heads = 0;
    if (in_lds) {
        {   // every source index first, then all loads in flight at once
            constexpr int kPer = kGdCap / kThreads;
            uint32_t src[kPer];
            uint64_t v[kPer];
#pragma unroll
            for (int j = 0; j < kPer; ++j) {
                const uint32_t k = tid + j * kThreads;
                src[j] = k < size ? src_of(k, s_map[k]) : 0u;
            }
#pragma unroll
            for (int j = 0; j < kPer; ++j)
                if (tid + j * kThreads < size) v[j] = tile_comp[src[j]];
#pragma unroll
            for (int j = 0; j < kPer; ++j)
                if (tid + j * kThreads < size) s_a[tid + j * kThreads] = v[j];
        }
        // buckets of the top sbits low key bits
        const int sbits = shift < kGdSubBits ? shift : kGdSubBits;
        const uint32_t nsub = 1u << sbits;
        const int sh = 32 + shift - sbits;
        auto sub = [&](uint64_t c) { return static_cast<uint32_t>(c >> sh) & (nsub - 1); };
        constexpr int kSubPer = kGdSub / kThreads;
#pragma unroll
        for (int q = 0; q < kSubPer; ++q) s_cur[tid * kSubPer + q] = 0u;
        __syncthreads();
        for (uint32_t k = tid; k < size; k += kThreads) atomicAdd(&s_cur[sub(s_a[k])], 1u);
        __syncthreads();
        {   // bucket starts: thread tid owns buckets [tid * kSubPer, tid * kSubPer + kSubPer)
            uint32_t c[kSubPer], sum = 0;
#pragma unroll
            for (int q = 0; q < kSubPer; ++q) {
                c[q] = s_cur[tid * kSubPer + q];
                sum += c[q];
            }
            uint32_t tot;
            uint32_t st = block_exclusive_scan(sum, s_wtot, &tot);
#pragma unroll
            for (int q = 0; q < kSubPer; ++q) {
                s_sb[tid * kSubPer + q] = st;
                s_cur[tid * kSubPer + q] = st;
                st += c[q];
            }
            if (tid == 0) s_sb[kGdSub] = size;
        }
        __syncthreads();
        for (uint32_t k = tid; k < size; k += kThreads) {
            const uint64_t c = s_a[k];
            s_b[atomicAdd(&s_cur[sub(c)], 1u)] = c;
        }
        __syncthreads();
        // rank inside the bucket (buckets past nsub are empty and start at size), four LDS
        // reads in flight per step, the last step masked; keys and positions compared as 32-bit
        // halves (a composite is less when its key is, or its key is equal and its position is)
        for (uint32_t k = tid; k < size; k += kThreads) {
            const uint64_t c = s_b[k];
            const uint32_t ck = static_cast<uint32_t>(c >> 32), cp = static_cast<uint32_t>(c);
            const uint32_t j = sub(c);
            const uint32_t blo = s_sb[j], bhi = s_sb[j + 1];
            uint32_t rank = 0, same = 0;
            auto count = [&](uint64_t dd) {
                const uint32_t dk = static_cast<uint32_t>(dd >> 32), dp = static_cast<uint32_t>(dd);
                rank += dk < ck ? 1u : 0u;
                same += (dk == ck && dp < cp) ? 1u : 0u;
            };
            uint32_t m = blo;
            for (; m + 16 <= bhi; m += 16) {  // a hot key's repeats: sixteen reads in flight
                uint64_t d[16];
#pragma unroll
                for (int q = 0; q < 16; ++q) d[q] = s_b[m + q];
#pragma unroll
                for (int q = 0; q < 16; ++q) count(d[q]);
            }
            for (; m < bhi; m += 4) {
                uint64_t d[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) d[q] = s_b[m + q < bhi ? m + q : k];  // k: never less
#pragma unroll
                for (int q = 0; q < 4; ++q) count(d[q]);
            }
            rank += same;
            s_a[blo + rank] = c;  // s_a is free again: every composite is in s_b
            heads += same == 0u ? 1u : 0u;
        }
        __syncthreads();
        for (uint32_t k = tid; k < size; k += kThreads) comp[gs + k] = s_a[k];
    } else {
        uint64_t *a = comp + gs;
        for (uint32_t k = tid; k < size; k += kThreads) {
            uint32_t lo_t = 0, hi_t = ntiles;  // s_run[lo_t] <= k < s_run[hi_t]
            while (hi_t - lo_t > 1) {
                const uint32_t m = (lo_t + hi_t) >> 1;
                if (s_run[m] <= k) lo_t = m; else hi_t = m;
            }
            a[k] = tile_comp[src_of(k, lo_t)];
        }
        __syncthreads();
        wg_radix_sort(a, tmp + gs, size, 32 + shift);
        for (uint32_t i = tid; i < size; i += kThreads)
            heads += (i == 0 || (a[i] >> 32) != (a[i - 1] >> 32)) ? 1u : 0u;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) heads += __shfl_xor(heads, o, 64);
    if (lane == 0) s_red[wave] = heads;
    __syncthreads();
    if (tid == 0) ucount[g] = s_red[0] + s_red[1] + s_red[2] + s_red[3];
}

// Group g: its unique keys numbered after the earlier groups' (a block sum over ucount[0, g));
// writes uniq, inv and the plan (spos, seg_start, seg_pos). The last group writes the count and the end
// of the last segment.
__global__ __launch_bounds__(kThreads) void gd_emit(const uint64_t *comp, const uint32_t *gstart,
                                                    const uint32_t *ucount, uint32_t ng, int shift,
                                                    int64_t *uniq, int64_t *inv, uint32_t *spos,
                                                    uint32_t *seg_start, uint32_t *seg_pos,
                                                    int64_t *count) {
    __shared__ uint64_t s_c[kGdCap];
    __shared__ uint32_t s_wtot[kThreads / 64];
    const int tid = threadIdx.x;
    const uint32_t g = blockIdx.x;
    const uint32_t lo = gstart[g], size = gstart[g + 1] - lo;
    const uint64_t gbase = static_cast<uint64_t>(g) << shift;
    const uint64_t *sorted = comp + lo;
    const bool in_lds = size <= static_cast<uint32_t>(kGdCap);
    if (in_lds) {  // the group's composites into LDS, every load in flight at once
        constexpr int kPer = kGdCap / kThreads;
        uint64_t v[kPer];
#pragma unroll
        for (int j = 0; j < kPer; ++j)
            if (tid + j * kThreads < size) v[j] = sorted[tid + j * kThreads];
#pragma unroll
        for (int j = 0; j < kPer; ++j)
            if (tid + j * kThreads < size) s_c[tid + j * kThreads] = v[j];
    }
    uint32_t prior = 0;
    for (uint32_t q = tid; q < g; q += kThreads) prior += ucount[q];
    uint32_t run;
    block_exclusive_scan(prior, s_wtot, &run);  // run = unique keys of the earlier groups (the
                                                // scan's barriers also publish s_c)
    if (g == ng - 1 && tid == 0) {
        const uint32_t total = run + ucount[g];
        *count = static_cast<int64_t>(total);
        seg_start[total] = lo + size;
    }
    // LDS and global memory through their own address spaces: one generic pointer for both would
    // compile to flat loads, whose aperture check sees the base before the instruction offset
    gmem_ptr<const uint64_t> gsorted = as_global(sorted);
    auto item = [&](uint32_t i) {
        uint64_t v;
        if (in_lds) v = s_c[i]; else v = gsorted[i];
        return v;
    };
    for (uint32_t c0 = 0; c0 < size; c0 += kThreads * kItems) {
        const uint32_t i0 = c0 + static_cast<uint32_t>(tid) * kItems;
        uint64_t v[kItems];
        bool head[kItems];
        uint32_t nh = 0;
        uint64_t prev = i0 > 0 && i0 < size ? item(i0 - 1) : ~0ull;
#pragma unroll
        for (int e = 0; e < kItems; ++e) {
            const uint32_t i = i0 + e;
            v[e] = i < size ? item(i) : ~0ull;
            head[e] = i < size && (i == 0 || (v[e] >> 32) != (prev >> 32));
            nh += head[e] ? 1u : 0u;
            prev = v[e];
        }
        uint32_t chunk_heads;
        uint32_t u = run + block_exclusive_scan(nh, s_wtot, &chunk_heads);
#pragma unroll
        for (int e = 0; e < kItems; ++e) {
            const uint32_t i = i0 + e;
            if (i < size) {
                const uint32_t pos = static_cast<uint32_t>(v[e]);
                if (head[e]) {
                    uniq[u] = static_cast<int64_t>(gbase + (v[e] >> 32));
                    seg_start[u] = lo + i;
                    seg_pos[u] = pos;
                    ++u;
                }
                inv[pos] = static_cast<int64_t>(u) - 1;
                spos[lo + i] = pos;
            }
        }
        run += chunk_heads;
    }
}

// ---- table dedup ------------------------------------------------------------------------------
// The key half of a row lookup's dedup when its keys come as per-table row ids: idx[k * stride +
// t] is the row of token t in table k (t < n), the key is offset_k + row and the lookup's
// position is t * nt + k (the token-major order of the gradient rows). Every table holds exactly
// n lookups, so in sorted key order table k's lookups fill [k * n, (k + 1) * n). Table k's rows
// are split into parts of 2^shift_k rows (part = row >> shift_k), and a part's place inside its
// table is the number of the table's lookups in lower parts -- which the part's workgroup counts
// itself while it reads the table's ids. So every part sorts its lookups where they land, with no
// exchange between workgroups; only the unique numbering needs the earlier parts' unique counts,
// which is the second launch:
//   td_part  per (table, part): the table's ids read once (two per thread per round of 512
//            tokens, all loads in flight) and kept as rows in LDS; one block scan counts the
//            part's lookups and the lookups of lower parts and gives each thread the slots of its
//            own, which it fills by walking its match bits; the composites (row in part, token)
//            are ranked inside 1024 buckets of their top row bits and written at the part's
//            place: spos (the position), and a slot copy (position, row) for td_emit; its size,
//            place and unique count into gsize, gstart and ucount. A part larger than LDS sorts
//            in global memory (stable LSD radix) and leaves its rows in srow.
//   td_emit  per (table, part): its unique keys numbered after the earlier parts' (a block sum
//            of their unique counts), then uniq, local rows, inv, the segment plan and the
//            table bounds (info = [count, first unique index of each table, count]).
constexpr uint32_t kTdMaxN = 8192;            // tokens per table this path takes
constexpr int kTdRounds = kTdMaxN / (2 * kThreads);  // 16: a thread's match bits fit 32
constexpr int kTdCap = 2048;                  // composites a part sorts in LDS
constexpr int kTdBucketBits = 10;
constexpr int kTdBuckets = 1 << kTdBucketBits;
constexpr int kTdPartTarget = 512;            // lookups per part aimed at

struct TdArgs {
    const int64_t *idx;
    int64_t stride;
    uint32_t n;
    int nt;
    uint32_t ngroups;
    int64_t rows[ME_MAX_TABLES];
    int64_t off[ME_MAX_TABLES];           // key offset of table k
    int32_t shift[ME_MAX_TABLES];         // log2 of a part's rows
    uint32_t gbase[ME_MAX_TABLES + 1];    // first part (group) of table k; gbase[nt] = ngroups
    uint32_t *spos, *seg_start, *seg_pos;  // the plan
    uint32_t *srow;                        // [n * nt] row of each lookup in sorted order (parts
                                           // larger than LDS)
    uint64_t *slot;                        // [ngroups * kTdCap] a part's sorted (position << 32 |
                                           // row), at a place known before the part's size
    uint64_t *tmp_a, *tmp_b;               // [n * nt] each: parts larger than LDS
    uint32_t *gstart, *gsize, *ucount;     // [ngroups]
    int64_t *uniq, *local, *inv, *info;
};

__device__ __forceinline__ int td_table_of(const TdArgs &a, uint32_t g) {
    int k = 0;
    while (k + 1 < a.nt && a.gbase[k + 1] <= g) ++k;
    return k;
}

// kRounds: rounds of 512 tokens the part's workgroup reads (a power of two, >= the table's n /
// 512); kVec2: two ids per 16-byte load (ids 16-byte aligned, stride and n even).
template <int kRounds, bool kVec2>
__global__ __launch_bounds__(kThreads) void td_part(const TdArgs a) {
    __shared__ uint64_t s_a[kTdCap];
    __shared__ uint64_t s_b[kTdCap];
    __shared__ uint32_t s_sb[kTdBuckets + 1];  // bucket starts
    __shared__ uint32_t s_cur[kTdBuckets];     // bucket fill counters
    __shared__ uint32_t s_wtot[kThreads / 64];
    __shared__ uint32_t s_red[kThreads / 64];
    __shared__ uint32_t s_rows[kTdMaxN];       // the table's rows, by token
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t g = blockIdx.x;
    const int k = td_table_of(a, g);
    const uint32_t part = g - a.gbase[k];
    const int sh = a.shift[k];
    const int64_t rmax = a.rows[k] - 1;
    const uint32_t n = a.n;
    const int64_t *ids = a.idx + static_cast<int64_t>(k) * a.stride;

    // ---- the table's ids: token t = r * 512 + 2 * tid + h, every load in flight at once. Rows
    // outside [0, rows) (outside the contract) are clamped, so nothing lands out of bounds.
    int64_t v[kRounds][2];
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
        const uint32_t t0 = static_cast<uint32_t>(r * 2 * kThreads + 2 * tid);
        if (kVec2) {
            u32x4_v w = u32x4_v{0u, 0u, 0u, 0u};
            if (t0 < n) w = *as_global(reinterpret_cast<const u32x4_v *>(ids + t0));
            v[r][0] = static_cast<int64_t>((static_cast<uint64_t>(w[1]) << 32) | w[0]);
            v[r][1] = static_cast<int64_t>((static_cast<uint64_t>(w[3]) << 32) | w[2]);
        } else {
            v[r][0] = t0 < n ? ids[t0] : 0;
            v[r][1] = t0 + 1 < n ? ids[t0 + 1] : 0;
        }
    }
    // each token's row (clamped) into LDS; bit 2r + h of `match` marks a lookup of this part
    // (kRounds <= 16: 32 bits); counts of this part's lookups and of lower parts'. A token past
    // n gets part ~0, which counts as neither.
    uint32_t match = 0;
    uint32_t cm = 0, cl = 0;
    const uint32_t rmax32 = static_cast<uint32_t>(rmax);
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
        uint32_t rw[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t t = static_cast<uint32_t>(r * 2 * kThreads + 2 * tid + h);
            const uint64_t x = static_cast<uint64_t>(v[r][h]);
            const uint32_t hi = static_cast<uint32_t>(x >> 32), lo = static_cast<uint32_t>(x);
            rw[h] = hi == 0u ? min(lo, rmax32) : (static_cast<int32_t>(hi) < 0 ? 0u : rmax32);
            const uint32_t p = t < n ? rw[h] >> sh : ~0u;
            const uint32_t mt = p == part ? 1u : 0u;
            cm += mt;
            cl += p < part ? 1u : 0u;
            match |= mt << (2 * r + h);
        }
        const uint32_t t0 = static_cast<uint32_t>(r * 2 * kThreads + 2 * tid);
        if (t0 < n) *reinterpret_cast<u32x2_v *>(&s_rows[t0]) = u32x2_v{rw[0], rw[1]};
    }
    // both counts in one block scan (each below 2^16: at most n <= 8192 of either); the low half
    // of this thread's exclusive prefix is where its own lookups of the part go
    uint32_t tot;
    const uint32_t pre = block_exclusive_scan((cl << 16) | cm, s_wtot, &tot);
    const uint32_t m = tot & 0xffffu;
    const uint32_t start = static_cast<uint32_t>(k) * n + (tot >> 16);
    const bool in_lds = m <= static_cast<uint32_t>(kTdCap);
    uint64_t *gbuf = a.tmp_a + start;
    // ---- the part's composites (row in part << 32 | token), each thread's at its own slots, in
    // no particular order (the sort below orders whole composites): one pass over the set bits
    const uint32_t lmask = (1u << sh) - 1u;
    uint32_t dst = pre & 0xffffu;
    while (match != 0u) {
        const int bit = __builtin_ctz(match);
        match &= match - 1u;
        const uint32_t t = static_cast<uint32_t>((bit >> 1) * 2 * kThreads + 2 * tid + (bit & 1));
        const uint64_t c = (static_cast<uint64_t>(s_rows[t] & lmask) << 32) | t;
        if (in_lds) s_a[dst] = c; else gbuf[dst] = c;
        ++dst;
    }
    __syncthreads();
    if (in_lds) {
        // buckets of the top row bits, then each composite ranked inside its bucket (composites
        // are distinct: the order of (row, token), i.e. the stable order of the keys)
        const int bbits = sh < kTdBucketBits ? sh : kTdBucketBits;
        const int bsh = 32 + sh - bbits;
        const uint32_t bmask = (1u << bbits) - 1u;
        auto bucket = [&](uint64_t c) { return static_cast<uint32_t>(c >> bsh) & bmask; };
        constexpr int kPer = kTdBuckets / kThreads;
#pragma unroll
        for (int q = 0; q < kPer; ++q) s_cur[tid * kPer + q] = 0u;
        __syncthreads();
        for (uint32_t i = tid; i < m; i += kThreads) atomicAdd(&s_cur[bucket(s_a[i])], 1u);
        __syncthreads();
        {
            uint32_t c[kPer], sum = 0;
#pragma unroll
            for (int q = 0; q < kPer; ++q) {
                c[q] = s_cur[tid * kPer + q];
                sum += c[q];
            }
            uint32_t btot;
            uint32_t st = block_exclusive_scan(sum, s_wtot, &btot);
#pragma unroll
            for (int q = 0; q < kPer; ++q) {
                s_sb[tid * kPer + q] = st;
                s_cur[tid * kPer + q] = st;
                st += c[q];
            }
            if (tid == 0) s_sb[kTdBuckets] = m;
        }
        __syncthreads();
        for (uint32_t i = tid; i < m; i += kThreads) {
            const uint64_t c = s_a[i];
            s_b[atomicAdd(&s_cur[bucket(c)], 1u)] = c;
        }
        __syncthreads();
        for (uint32_t i = tid; i < m; i += kThreads) {
            const uint64_t c = s_b[i];
            const uint32_t j = bucket(c);
            const uint32_t blo = s_sb[j], bhi = s_sb[j + 1];
            uint32_t rank = 0;
            uint32_t q = blo;
            for (; q + 8 <= bhi; q += 8) {  // a hot row's repeats: eight reads in flight
                uint64_t d[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) d[e] = s_b[q + e];
#pragma unroll
                for (int e = 0; e < 8; ++e) rank += d[e] < c ? 1u : 0u;
            }
            for (; q < bhi; ++q) rank += s_b[q] < c ? 1u : 0u;
            s_a[blo + rank] = c;
        }
        __syncthreads();
    } else {
        wg_radix_sort(gbuf, a.tmp_b + start, m, 32 + sh);
    }
    // ---- the part's lookups at its place: position and row; its unique count. LDS and global
    // memory are read through their own pointers: a generic pointer into LDS let the compiler
    // form sorted + i - 1 as an address below the LDS aperture (s_a sits at LDS offset 0) with
    // the 8 bytes in the instruction offset, and the aperture is checked on that base.
    uint32_t heads = 0;
    const uint32_t rbase = part << sh;
    uint64_t *slot = a.slot + static_cast<uint64_t>(g) * kTdCap;
    auto put = [&](uint32_t i, uint64_t c, uint64_t prev) {
        const uint32_t rl = static_cast<uint32_t>(c >> 32), t = static_cast<uint32_t>(c);
        heads += (i == 0 || static_cast<uint32_t>(prev >> 32) != rl) ? 1u : 0u;
        const uint32_t pos = t * static_cast<uint32_t>(a.nt) + static_cast<uint32_t>(k);
        a.spos[start + i] = pos;
        if (in_lds) slot[i] = (static_cast<uint64_t>(pos) << 32) | (rbase + rl);
        else a.srow[start + i] = rbase + rl;
    };
    if (in_lds) {
        for (uint32_t i = tid; i < m; i += kThreads) put(i, s_a[i], s_a[i > 0 ? i - 1 : 0]);
    } else {
        gmem_ptr<const uint64_t> gs = as_global(static_cast<const uint64_t *>(gbuf));
        for (uint32_t i = tid; i < m; i += kThreads) put(i, gs[i], gs[i > 0 ? i - 1 : 0]);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) heads += __shfl_xor(heads, o, 64);
    if (lane == 0) s_red[wave] = heads;
    __syncthreads();
    if (tid == 0) {
        a.gstart[g] = start;
        a.gsize[g] = m;
        a.ucount[g] = s_red[0] + s_red[1] + s_red[2] + s_red[3];
    }
}

__global__ __launch_bounds__(kThreads) void td_emit(const TdArgs a) {
    __shared__ uint32_t s_wtot[kThreads / 64];
    const int tid = threadIdx.x;
    const uint32_t g = blockIdx.x;
    const int k = td_table_of(a, g);
    const bool last = g + 1 == a.ngroups;
    // every first load at once: the part's place and size, the earlier parts' unique counts, and
    // the part's sorted lookups from its slot (a part that fit LDS left them there; thread tid owns
    // [8 tid, 8 tid + 8) and reads the one before)
    const uint32_t lo = a.gstart[g], size = a.gsize[g];
    const uint64_t *slot = a.slot + static_cast<uint64_t>(g) * kTdCap;
    uint64_t sv[kItems + 1];
    sv[0] = tid > 0 ? slot[tid * kItems - 1] : 0ull;
#pragma unroll
    for (int e = 0; e < kItems; ++e) sv[e + 1] = slot[tid * kItems + e];
    const uint32_t lim = last ? a.ngroups : g;
    uint32_t before = 0, all = 0;
    for (uint32_t q0 = 0; q0 < lim; q0 += kThreads * 8) {
        uint32_t c[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t q = q0 + e * kThreads + tid;
            c[e] = q < lim ? a.ucount[q] : 0u;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t q = q0 + e * kThreads + tid;
            before += q < g ? c[e] : 0u;
            all += c[e];
        }
    }
    uint32_t run, total;
    block_exclusive_scan(before, s_wtot, &run);
    block_exclusive_scan(all, s_wtot, &total);
    if (tid == 0) {
        if (g == a.gbase[k]) a.info[1 + k] = static_cast<int64_t>(run);
        if (last) {
            a.info[0] = static_cast<int64_t>(total);
            a.info[1 + a.nt] = static_cast<int64_t>(total);
            a.seg_start[total] = a.n * static_cast<uint32_t>(a.nt);
        }
    }
    const int64_t off = a.off[k];
    const bool from_slot = size <= static_cast<uint32_t>(kTdCap);
    for (uint32_t c0 = 0; c0 < size; c0 += kThreads * kItems) {
        const uint32_t i0 = c0 + static_cast<uint32_t>(tid) * kItems;
        uint32_t r[kItems], p[kItems];
        uint32_t prev;
        if (from_slot) {  // one chunk: size <= kTdCap = kThreads * kItems
            prev = static_cast<uint32_t>(sv[0]);
#pragma unroll
            for (int e = 0; e < kItems; ++e) {
                r[e] = static_cast<uint32_t>(sv[e + 1]);
                p[e] = static_cast<uint32_t>(sv[e + 1] >> 32);
            }
        } else {
            prev = i0 > 0 && i0 < size ? a.srow[lo + i0 - 1] : 0u;
#pragma unroll
            for (int e = 0; e < kItems; ++e) {
                const uint32_t i = i0 + e;
                r[e] = i < size ? a.srow[lo + i] : 0u;
                p[e] = i < size ? a.spos[lo + i] : 0u;
            }
        }
        bool head[kItems];
        uint32_t nh = 0;
#pragma unroll
        for (int e = 0; e < kItems; ++e) {
            const uint32_t i = i0 + e;
            head[e] = i < size && (i == 0 || r[e] != prev);
            nh += head[e] ? 1u : 0u;
            prev = r[e];
        }
        uint32_t chunk_heads;
        uint32_t u = run + block_exclusive_scan(nh, s_wtot, &chunk_heads);
#pragma unroll
        for (int e = 0; e < kItems; ++e) {
            const uint32_t i = i0 + e;
            if (i < size) {
                if (head[e]) {
                    a.uniq[u] = off + r[e];
                    a.local[u] = r[e];
                    a.seg_start[u] = lo + i;
                    a.seg_pos[u] = p[e];
                    ++u;
                }
                if (a.inv != nullptr) a.inv[p[e]] = static_cast<int64_t>(u) - 1;
            }
        }
        run += chunk_heads;
    }
}

// A table's part width: the smallest 2^shift rows for which the table has at most `target`
// parts (shift <= 31, so a row inside its part fits the 32 bits of a composite).
int td_shift(int64_t rows, int64_t target) {
    int s = 0;
    while (s < 31 && ((rows - 1) >> s) + 1 > target) ++s;
    return s;
}

// ---- squared norm ---------------------------------------------------------------------------
constexpr int kSumBlocks = 256;
constexpr int kSumThreads = 1024;
constexpr int kSumLoads = 8;  // the accumulator tree below adds eight

// Partial sums of x^2: thread t of block b owns elements b * kSumThreads + t + k * step (step =
// kSumBlocks * kSumThreads), eight of them in flight at a time into eight accumulators (k mod
// 8) combined in a fixed tree; the block's threads are added in a fixed tree, and one workgroup
// adds the kSumBlocks partials in order. The order is fixed, so the result is deterministic.
// (One 256-thread block per CU with one load in flight per thread read 47 MB at ~1 TB/s.)
__global__ __launch_bounds__(kSumThreads) void sumsq_partial(const float *x, int64_t n, float *partial) {
    __shared__ float s[kSumThreads];
    const int tid = threadIdx.x;
    constexpr int64_t kStep = static_cast<int64_t>(kSumBlocks) * kSumThreads;
    float acc[kSumLoads];
#pragma unroll
    for (int u = 0; u < kSumLoads; ++u) acc[u] = 0.f;
    int64_t i = static_cast<int64_t>(blockIdx.x) * kSumThreads + tid;
    for (; i + (kSumLoads - 1) * kStep < n; i += kSumLoads * kStep) {
        float v[kSumLoads];
#pragma unroll
        for (int u = 0; u < kSumLoads; ++u) v[u] = x[i + u * kStep];
#pragma unroll
        for (int u = 0; u < kSumLoads; ++u) acc[u] += v[u] * v[u];
    }
#pragma unroll
    for (int u = 0; u < kSumLoads - 1; ++u)  // fewer than kSumLoads elements left
        if (i + u * kStep < n) acc[u] += x[i + u * kStep] * x[i + u * kStep];
    s[tid] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    __syncthreads();
    for (int off = kSumThreads / 2; off > 0; off >>= 1) {
        if (tid < off) s[tid] += s[tid + off];
        __syncthreads();
    }
    if (tid == 0) partial[blockIdx.x] = s[0];
}

__global__ __launch_bounds__(kSumBlocks) void sumsq_final(const float *partial, float *out, int accumulate) {
    __shared__ float s[kSumBlocks];
    const int tid = threadIdx.x;
    s[tid] = partial[tid];
    __syncthreads();
    for (int off = kSumBlocks / 2; off > 0; off >>= 1) {
        if (tid < off) s[tid] += s[tid + off];
        __syncthreads();
    }
    if (tid == 0) *out = accumulate ? *out + s[0] : s[0];
}

// ---- clip: scale the gradients in place -------------------------------------------------------
// RowTables.clip (rows.py:221-231): norm = sqrt(sumsq); coef = max_norm / (norm + 1e-6), which
// torch evaluates as Tensor.__rtruediv__, i.e. reciprocal(norm + 1e-6) * max_norm, in fp32, then
// clamp(max=1) (a NaN coef stays NaN); fp32 x *= coef, bf16 x *= coef rounded to bf16 first
// (p.grad.mul_(coef.to(p.grad.dtype))), the product rounded to bf16. Every thread computes the
// coefficient from the device scalar itself, so the host never reads the norm for this.
__device__ __forceinline__ float clip_coef(const float *sumsq, float max_norm) {
    const float r = 1.0f / (sqrtf(*sumsq) + 1e-6f);  // correctly rounded division and sqrt
    const float c = r * max_norm;
    return c > 1.0f ? 1.0f : c;
}

constexpr int kClipThreads = 256;

// fp32: 4 values per 16-byte load; bf16: 8. Grid-stride over vectors, then a scalar tail.
template <bool BF16>
__global__ __launch_bounds__(kClipThreads) void clip_scale(void *x, int64_t n, const float *sumsq,
                                                           float max_norm) {
    float coef = clip_coef(sumsq, max_norm);
    if (BF16) coef = round_to_bf16(coef);
    constexpr int kPer = BF16 ? 8 : 4;
    const int64_t nvec = n / kPer;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kClipThreads;
    int64_t i = static_cast<int64_t>(blockIdx.x) * kClipThreads + threadIdx.x;
    gmem_ptr<u32x4_v> xv = as_global(reinterpret_cast<u32x4_v *>(x));
    for (; i < nvec; i += stride) {
        u32x4_v w = xv[i];
        if (BF16) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float lo = __uint_as_float(w[q] << 16) * coef;
                const float hi = __uint_as_float(w[q] & 0xffff0000u) * coef;
                w[q] = static_cast<uint32_t>(float_to_bf16_bits_rne(lo)) |
                       (static_cast<uint32_t>(float_to_bf16_bits_rne(hi)) << 16);
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) w[q] = __float_as_uint(__uint_as_float(w[q]) * coef);
        }
        xv[i] = w;
    }
    // the last n % kPer values: one thread each, in the first block
    if (blockIdx.x == 0 && threadIdx.x < n - nvec * kPer) {
        const int64_t j = nvec * kPer + threadIdx.x;
        if (BF16) {
            uint16_t *xb = static_cast<uint16_t *>(x);
            xb[j] = float_to_bf16_bits_rne(bf16_bits_to_float(xb[j]) * coef);
        } else {
            float *xf = static_cast<float *>(x);
            xf[j] = xf[j] * coef;
        }
    }
}

// ---- Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11) ----------------------------------------
__device__ __forceinline__ uint4 philox4x32_10(uint4 c, uint2 k) {
    constexpr uint32_t kM0 = 0xD2511F53u, kM1 = 0xCD9E8D57u;
    constexpr uint32_t kW0 = 0x9E3779B9u, kW1 = 0xBB67AE85u;
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        // one 32 x 32 -> 64-bit product per word gives both halves (v_mad_u64_u32)
        const uint64_t p0 = static_cast<uint64_t>(kM0) * c.x, p1 = static_cast<uint64_t>(kM1) * c.z;
        c = make_uint4(static_cast<uint32_t>(p1 >> 32) ^ c.y ^ k.x, static_cast<uint32_t>(p1),
                       static_cast<uint32_t>(p0 >> 32) ^ c.w ^ k.y, static_cast<uint32_t>(p0));
        k.x += kW0;
        k.y += kW1;
    }
    return c;
}

// 16 bits of rounding noise for element (row, col) of array `which` (0: weights, 1: first
// moment, 2: per-value second moment) of table `table` at step `step`.
__device__ __forceinline__ uint32_t sr_noise(uint64_t seed, uint32_t step, uint32_t table,
                                             uint64_t row, uint32_t col, uint32_t which) {
    const uint4 ctr = make_uint4(static_cast<uint32_t>(row), static_cast<uint32_t>(row >> 32), step,
                                 (table << 16) | (which << 14) | (col >> 3));
    const uint4 w = philox4x32_10(ctr, make_uint2(static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32)));
    const uint32_t sel = (col >> 1) & 3;
    const uint32_t word = sel == 0 ? w.x : sel == 1 ? w.y : sel == 2 ? w.z : w.w;
    return (word >> (16 * (col & 1))) & 0xffffu;
}

// fp32 -> bf16 bits, stochastic: noise added below the kept 16 bits, then truncated; inf and NaN
// convert as usual (optim.py:39-44).
__device__ __forceinline__ uint16_t stochastic_bf16_bits(float x, uint32_t noise) {
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7f800000u) == 0x7f800000u) return float_to_bf16_bits_rne(x);
    return static_cast<uint16_t>((u + noise) >> 16);
}

// ---- lazy / row-wise Adam on touched rows ------------------------------------------------------
struct AdamTable {
    uint8_t *param;        // [rows, dim] of the parameter dtype
    uint8_t *exp_avg;      // like param
    uint8_t *exp_avg_sq;   // row-wise: [rows] fp32; per value: like param
    const int64_t *rows;   // [n] unique row ids
    const uint8_t *grads;  // [n, dim] fp32 or bf16 (grad_bf16)
    int64_t n;
    int64_t first;         // first global row slot of this table in the launch
    float neg_lr_bc1;      // -lr / (1 - beta1^step)
    float sqrt_bc2;        // sqrt(1 - beta2^step)
    uint32_t step;
    uint32_t stream_id;    // RNG stream of this table
};

constexpr int kAdamTables = 32;  // tables per launch (kernel arguments stay under 4 KiB)

struct AdamArgs {
    AdamTable t[kAdamTables];
    int n_tables;
    int64_t total;
    int dim;
    int param_bf16;
    int rowwise;
    int sq_bf16;           // per-value second moment stored as bf16
    int grad_bf16;         // gradient rows stored as bf16
    int sr;
    int lazy;              // skip rows whose gradient is all zero
    uint64_t seed;
    float decay;           // 1 - lr * weight_decay (1: no decay)
    int has_decay;
    float beta1, one_minus_beta1, beta2, one_minus_beta2, eps;
};

__device__ __forceinline__ float load_elem(const uint8_t *base, int bf16, int64_t i) {
    return bf16 ? bf16_bits_to_float(reinterpret_cast<const uint16_t *>(base)[i])
                : reinterpret_cast<const float *>(base)[i];
}

__device__ __forceinline__ void store_elem(uint8_t *base, int bf16, int64_t i, float v, int sr,
                                           uint32_t noise) {
    if (bf16)
        reinterpret_cast<uint16_t *>(base)[i] = sr ? stochastic_bf16_bits(v, noise) : float_to_bf16_bits_rne(v);
    else
        reinterpret_cast<float *>(base)[i] = v;
}

// One wave per touched row; lane c holds columns c, c + 64, ... of the row.
__global__ __launch_bounds__(kThreads) void adam_rows(const AdamArgs a) {
    const int lane = threadIdx.x & 63;
    const int64_t slot = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
    if (slot >= a.total) return;
    int k = 0;
    while (k + 1 < a.n_tables && a.t[k + 1].first <= slot) ++k;
    const AdamTable &t = a.t[k];
    const int64_t i = slot - t.first;
    const int64_t row = *as_global(t.rows + i);
    const int D = a.dim;
    const int64_t g_row = i * D;
    // lazy: a row whose gradient is all zero is skipped entirely (optim.py:92-95)
    bool any = false;
    float gsq = 0.f;
    for (int c = lane; c < D; c += 64) {
        const float g = load_elem(t.grads, a.grad_bf16, g_row + c);
        any |= g != 0.f;
        gsq += g * g;
    }
    if (a.lazy && __ballot(any) == 0ull) return;
    if (a.rowwise) {
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) gsq += __shfl_xor(gsq, off, 64);
    }

    const int64_t prow = row * D;
    float v_row = 0.f, denom_row = 0.f;
    if (a.rowwise) {
        const float v = *as_global(reinterpret_cast<const float *>(t.exp_avg_sq) + row);
        v_row = fmaf(gsq / static_cast<float>(D), a.one_minus_beta2, v * a.beta2);
        denom_row = sqrtf(v_row) / t.sqrt_bc2 + a.eps;
    }
    for (int c = lane; c < D; c += 64) {
        const float g = load_elem(t.grads, a.grad_bf16, g_row + c);
        float p = load_elem(t.param, a.param_bf16, prow + c);
        float m = load_elem(t.exp_avg, a.param_bf16, prow + c);
        if (a.has_decay) p = p * a.decay;
        m = fmaf(g, a.one_minus_beta1, m * a.beta1);
        float denom;
        if (a.rowwise) {
            denom = denom_row;
        } else {
            float v = load_elem(t.exp_avg_sq, a.sq_bf16, prow + c);
            v = v * a.beta2 + a.one_minus_beta2 * g * g;
            denom = sqrtf(v) / t.sqrt_bc2 + a.eps;
            const uint32_t nv = a.sr && a.sq_bf16 ? sr_noise(a.seed, t.step, t.stream_id, row, c, 2) : 0u;
            store_elem(t.exp_avg_sq, a.sq_bf16, prow + c, v, a.sr, nv);
        }
        p = p + (t.neg_lr_bc1 * m) / denom;
        const bool rnd = a.sr && a.param_bf16;
        store_elem(t.param, a.param_bf16, prow + c, p, a.sr,
                   rnd ? sr_noise(a.seed, t.step, t.stream_id, row, c, 0) : 0u);
        store_elem(t.exp_avg, a.param_bf16, prow + c, m, a.sr,
                   rnd ? sr_noise(a.seed, t.step, t.stream_id, row, c, 1) : 0u);
    }
    if (a.rowwise && lane == 0) *as_global(reinterpret_cast<float *>(t.exp_avg_sq) + row) = v_row;
}

// C consecutive columns c0 .. c0 + C - 1 (C = 4 or 8, c0 % C == 0) take their noise from one
// Philox call: the same noise sr_noise gives each of them (word (col >> 1) & 3, half col & 1
// of the call for col >> 3); eight columns use all four words of the call.
template <int C>
__device__ __forceinline__ void sr_noise_cols(uint64_t seed, uint32_t step, uint32_t table,
                                              uint64_t row, uint32_t c0, uint32_t which,
                                              uint32_t (&nz)[C]) {
    const uint4 ctr = make_uint4(static_cast<uint32_t>(row), static_cast<uint32_t>(row >> 32), step,
                                 (table << 16) | (which << 14) | (c0 >> 3));
    const uint4 w = philox4x32_10(ctr, make_uint2(static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32)));
    uint32_t words[C / 2];
    if constexpr (C == 8) {
        words[0] = w.x; words[1] = w.y; words[2] = w.z; words[3] = w.w;
    } else {
        const bool low = ((c0 >> 1) & 3) == 0;
        words[0] = low ? w.x : w.z;
        words[1] = low ? w.y : w.w;
    }
#pragma unroll
    for (int j = 0; j < C; ++j) nz[j] = (words[j >> 1] >> (16 * (j & 1))) & 0xffffu;
}

// Nontemporal loads and stores: the sparse update reads and writes each touched row once, so
// its weight, moment and gradient lines are not kept in the caches (where they would only evict
// other rows' lines); on the update of 196,608 lookups this takes row-wise Adam from 52 to 36
// us. The 4-byte row-wise second moments and the row ids stay cached: nontemporal access
// there measured 9 us slower.
template <typename T>
__device__ __forceinline__ T ld_nt(const T *p) {
    return __builtin_nontemporal_load(as_global(p));
}

template <typename T>
__device__ __forceinline__ void st_nt(T *p, T v) {
    __builtin_nontemporal_store(v, as_global(p));
}

// Columns e0 .. e0 + C - 1 of an fp32 or bf16 array as fp32 (one 8- or 16-byte load for bf16,
// C / 4 16-byte loads for fp32), nontemporal.
template <int C, bool BF16>
__device__ __forceinline__ void load_cols(const uint8_t *base, int64_t e0, float (&x)[C]) {
    if constexpr (BF16) {
        uint32_t h[C / 2];
        if constexpr (C == 8) {
            const u32x4_v v = ld_nt(reinterpret_cast<const u32x4_v *>(base + e0 * 2));
            h[0] = v.x; h[1] = v.y; h[2] = v.z; h[3] = v.w;
        } else {
            const u32x2_v v = ld_nt(reinterpret_cast<const u32x2_v *>(base + e0 * 2));
            h[0] = v.x; h[1] = v.y;
        }
#pragma unroll
        for (int j = 0; j < C; ++j) x[j] = bf16_bits_to_float(static_cast<uint16_t>(h[j >> 1] >> (16 * (j & 1))));
    } else {
#pragma unroll
        for (int q = 0; q < C / 4; ++q) {
            const f32x4_v v = ld_nt(reinterpret_cast<const f32x4_v *>(base + (e0 + 4 * q) * 4));
            x[4 * q] = v.x; x[4 * q + 1] = v.y; x[4 * q + 2] = v.z; x[4 * q + 3] = v.w;
        }
    }
}

template <int C, bool BF16>
__device__ __forceinline__ void store_cols(uint8_t *base, int64_t e0, const float (&x)[C], int sr,
                                           const uint32_t (&nz)[C]) {
    if constexpr (BF16) {
        uint32_t h[C];
#pragma unroll
        for (int j = 0; j < C; ++j)
            h[j] = sr ? stochastic_bf16_bits(x[j], nz[j]) : float_to_bf16_bits_rne(x[j]);
        if constexpr (C == 8)
            st_nt(reinterpret_cast<u32x4_v *>(base + e0 * 2),
                  u32x4_v{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)});
        else
            st_nt(reinterpret_cast<u32x2_v *>(base + e0 * 2), u32x2_v{h[0] | (h[1] << 16), h[2] | (h[3] << 16)});
    } else {
#pragma unroll
        for (int q = 0; q < C / 4; ++q)
            st_nt(reinterpret_cast<f32x4_v *>(base + (e0 + 4 * q) * 4),
                  f32x4_v{x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]});
    }
}

// LPR lanes per touched row, C columns per lane (dim = C * LPR), 64 / LPR rows per wave: the
// same update as adam_rows with vector loads, one Philox call per lane per rounded array, and
// the launch's table list staged in LDS (rows of one wave may belong to different tables). The
// row's weights and moments are loaded together with its gradient, before the lazy test, so
// that one memory round trip follows the row id's. The weight dtype (PB: bf16, else fp32) and
// the second-moment form (RW: one fp32 per row) are template parameters: a run-time branch
// around each load makes the compiler wait for every load before issuing the next. So is the
// gradients' dtype (GB: bf16, else fp32).
template <int LPR, int C, bool PB, bool RW, bool GB>
__global__ __launch_bounds__(kThreads) void adam_rows_vec(const AdamArgs a) {
    constexpr int kRowsPerWave = 64 / LPR;
    constexpr int kRowsPerBlock = kRowsPerWave * (kThreads / 64);
    constexpr int D = C * LPR;
    __shared__ AdamTable s_t[kAdamTables];
    const int tid = threadIdx.x;
    {
        static_assert(sizeof(AdamTable) % 8 == 0, "table record copied as 8-byte words");
        const uint64_t *src = reinterpret_cast<const uint64_t *>(a.t);
        uint64_t *dst = reinterpret_cast<uint64_t *>(s_t);
        const int words = a.n_tables * static_cast<int>(sizeof(AdamTable) / 8);
        for (int w = tid; w < words; w += kThreads) dst[w] = src[w];
    }
    __syncthreads();
    const int lane = tid & 63;
    const int sub = lane & (LPR - 1);
    const int64_t slot = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (tid >> 6) * kRowsPerWave +
                         lane / LPR;
    if (slot >= a.total) return;  // whole rows: the lanes of one row share the slot
    int lo = 0, hi = a.n_tables - 1;  // last table whose first slot is <= slot
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_t[mid].first <= slot) lo = mid; else hi = mid - 1;
    }
    const AdamTable &t = s_t[lo];
    const int c0 = C * sub;
    const int64_t i = slot - t.first;
    float g[C], p[C], m[C], v[C];
    load_cols<C, GB>(t.grads, i * D + c0, g);
    const int64_t row = *as_global(t.rows + i);
    const int64_t e0 = row * D + c0;
    load_cols<C, PB>(t.param, e0, p);
    load_cols<C, PB>(t.exp_avg, e0, m);
    float v0 = 0.f;
    if constexpr (RW)
        v0 = *as_global(reinterpret_cast<const float *>(t.exp_avg_sq) + row);
    else if (a.sq_bf16)
        load_cols<C, true>(t.exp_avg_sq, e0, v);
    else
        load_cols<C, false>(t.exp_avg_sq, e0, v);
    bool any = false;
    float gsq = 0.f;
#pragma unroll
    for (int e = 0; e < C; ++e) {
        any |= g[e] != 0.f;
        gsq += g[e] * g[e];
    }
    // lazy: a row whose gradient is all zero is skipped entirely (optim.py:92-95)
    const uint64_t mask = __ballot(any);
    const uint64_t row_bits = LPR == 64 ? mask : (mask >> ((lane / LPR) * LPR)) & ((1ull << (LPR & 63)) - 1);
    if (a.lazy && row_bits == 0ull) return;
    if constexpr (RW) {
#pragma unroll
        for (int off = LPR / 2; off >= 1; off >>= 1) gsq += __shfl_xor(gsq, off, 64);
    }
    float v_row = 0.f, denom_row = 0.f;
    if constexpr (RW) {
        v_row = fmaf(gsq / static_cast<float>(D), a.one_minus_beta2, v0 * a.beta2);
        denom_row = sqrtf(v_row) / t.sqrt_bc2 + a.eps;
    }
#pragma unroll
    for (int e = 0; e < C; ++e) {
        if (a.has_decay) p[e] = p[e] * a.decay;
        m[e] = fmaf(g[e], a.one_minus_beta1, m[e] * a.beta1);
        float denom = denom_row;
        if constexpr (!RW) {
            v[e] = v[e] * a.beta2 + a.one_minus_beta2 * g[e] * g[e];
            denom = sqrtf(v[e]) / t.sqrt_bc2 + a.eps;
        }
        p[e] = p[e] + (t.neg_lr_bc1 * m[e]) / denom;
    }
    uint32_t nz[C];
#pragma unroll
    for (int e = 0; e < C; ++e) nz[e] = 0u;
    if constexpr (!RW) {
        if (a.sq_bf16) {
            if (a.sr) sr_noise_cols<C>(a.seed, t.step, t.stream_id, row, c0, 2, nz);
            store_cols<C, true>(t.exp_avg_sq, e0, v, a.sr, nz);
        } else {
            store_cols<C, false>(t.exp_avg_sq, e0, v, a.sr, nz);
        }
    }
    const bool rnd = PB && a.sr;
    if (rnd) sr_noise_cols<C>(a.seed, t.step, t.stream_id, row, c0, 0, nz);
    store_cols<C, PB>(t.param, e0, p, a.sr, nz);
    if (rnd) sr_noise_cols<C>(a.seed, t.step, t.stream_id, row, c0, 1, nz);
    store_cols<C, PB>(t.exp_avg, e0, m, a.sr, nz);
    if (RW && sub == 0) *as_global(reinterpret_cast<float *>(t.exp_avg_sq) + row) = v_row;
}

// Rows wider than 64 lanes x C columns (the dense key / value weights: 1,536 columns): one wave
// per row walking nb blocks of 64 x C columns, the same arithmetic and noise as adam_rows_vec per
// block. The lazy skip and the row-wise second moment need the whole row's gradient first: a
// pass over its blocks before the update pass (which loads them again).
template <int C, bool PB, bool RW, bool GB>
__global__ __launch_bounds__(kThreads) void adam_rows_wide(const AdamArgs a) {
    __shared__ AdamTable s_t[kAdamTables];
    const int tid = threadIdx.x;
    {
        const uint64_t *src = reinterpret_cast<const uint64_t *>(a.t);
        uint64_t *dst = reinterpret_cast<uint64_t *>(s_t);
        const int words = a.n_tables * static_cast<int>(sizeof(AdamTable) / 8);
        for (int w = tid; w < words; w += kThreads) dst[w] = src[w];
    }
    __syncthreads();
    const int lane = tid & 63;
    const int64_t slot = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (tid >> 6);
    if (slot >= a.total) return;
    int lo = 0, hi = a.n_tables - 1;  // last table whose first slot is <= slot
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_t[mid].first <= slot) lo = mid; else hi = mid - 1;
    }
    const AdamTable &t = s_t[lo];
    const int D = a.dim, nb = D / (64 * C);
    const int64_t i = slot - t.first;
    const int64_t row = *as_global(t.rows + i);
    const uint8_t *grow = t.grads;
    float v_row = 0.f, denom_row = 0.f;
    if (RW || a.lazy) {
        bool any = false;
        float gsq = 0.f;
        for (int b = 0; b < nb; ++b) {
            float g[C];
            load_cols<C, GB>(grow, i * D + b * 64 * C + lane * C, g);
#pragma unroll
            for (int e = 0; e < C; ++e) {
                any |= g[e] != 0.f;
                gsq += g[e] * g[e];
            }
        }
        // lazy: a row whose gradient is all zero is skipped entirely (optim.py:92-95)
        if (a.lazy && __ballot(any) == 0ull) return;
        if constexpr (RW) {
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) gsq += __shfl_xor(gsq, off, 64);
            const float v0 = *as_global(reinterpret_cast<const float *>(t.exp_avg_sq) + row);
            v_row = fmaf(gsq / static_cast<float>(D), a.one_minus_beta2, v0 * a.beta2);
            denom_row = sqrtf(v_row) / t.sqrt_bc2 + a.eps;
        }
    }
    for (int b = 0; b < nb; ++b) {
        const int c0 = b * 64 * C + lane * C;
        const int64_t e0 = row * D + c0;
        float g[C], p[C], m[C], v[C];
        load_cols<C, GB>(grow, i * D + c0, g);
        load_cols<C, PB>(t.param, e0, p);
        load_cols<C, PB>(t.exp_avg, e0, m);
        if constexpr (!RW) {
            if (a.sq_bf16)
                load_cols<C, true>(t.exp_avg_sq, e0, v);
            else
                load_cols<C, false>(t.exp_avg_sq, e0, v);
        }
#pragma unroll
        for (int e = 0; e < C; ++e) {
            if (a.has_decay) p[e] = p[e] * a.decay;
            m[e] = fmaf(g[e], a.one_minus_beta1, m[e] * a.beta1);
            float denom = denom_row;
            if constexpr (!RW) {
                v[e] = v[e] * a.beta2 + a.one_minus_beta2 * g[e] * g[e];
                denom = sqrtf(v[e]) / t.sqrt_bc2 + a.eps;
            }
            p[e] = p[e] + (t.neg_lr_bc1 * m[e]) / denom;
        }
        uint32_t nz[C];
#pragma unroll
        for (int e = 0; e < C; ++e) nz[e] = 0u;
        if constexpr (!RW) {
            if (a.sq_bf16) {
                if (a.sr) sr_noise_cols<C>(a.seed, t.step, t.stream_id, row, c0, 2, nz);
                store_cols<C, true>(t.exp_avg_sq, e0, v, a.sr, nz);
            } else {
                store_cols<C, false>(t.exp_avg_sq, e0, v, a.sr, nz);
            }
        }
        const bool rnd = PB && a.sr;
        if (rnd) sr_noise_cols<C>(a.seed, t.step, t.stream_id, row, c0, 0, nz);
        store_cols<C, PB>(t.param, e0, p, a.sr, nz);
        if (rnd) sr_noise_cols<C>(a.seed, t.step, t.stream_id, row, c0, 1, nz);
        store_cols<C, PB>(t.exp_avg, e0, m, a.sr, nz);
    }
    if (RW && lane == 0) *as_global(reinterpret_cast<float *>(t.exp_avg_sq) + row) = v_row;
}

// Standalone stochastic rounding of n fp32 values; element i uses the noise of (row i / 4096,
// column i % 4096) of stream `stream_id` at step `step`, array 0.
__global__ __launch_bounds__(kThreads) void sr_convert(const float *x, int64_t n, uint16_t *out,
                                                       uint64_t seed, uint32_t step, uint32_t stream_id) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= n) return;
    const uint64_t row = static_cast<uint64_t>(i) >> 12;
    const uint32_t col = static_cast<uint32_t>(i & 4095);
    out[i] = stochastic_bf16_bits(x[i], sr_noise(seed, step, stream_id, row, col, 0));
}

int sort_bits(int64_t key_bound) {
    int bits = 1;
    while (bits < 63 && (int64_t{1} << bits) < key_bound) ++bits;
    return bits;
}

struct DedupLayout {
    int nblocks, hist_stride;
    uint32_t ng_max;  // groups the group dedup may use (0: it is not used for this n)
    uint32_t ntiles;  // its tiles
    size_t keys_b, pos_a, pos_b, hist, heads, seg_start, seg_pos, tmp, gd_off, gd_start, gd_ucount, total;
};

// The group dedup is used up to kGdMaxN keys (kGdMaxTiles tiles of kGdTile).
constexpr int64_t kGdMaxN = static_cast<int64_t>(kGdMaxTiles) * kGdTile;

DedupLayout dedup_layout(int64_t n) {
    DedupLayout l{};
    l.nblocks = static_cast<int>(ceil_div(n, kTile));
    if (n <= kGdMaxN) {
        l.ng_max = static_cast<uint32_t>(std::min<int64_t>(n / kGdMean + 1, kGdMaxGroups));
        l.ntiles = static_cast<uint32_t>(ceil_div(n, kGdTile));
    }
    auto up = [](size_t x) { return (x + 255) & ~size_t{255}; };
    size_t off = 0;
    l.keys_b = off; off += up(static_cast<size_t>(n) * 8 * 2);  // two key buffers
    l.pos_a = off; off += up(static_cast<size_t>(n) * 4);
    l.pos_b = off; off += up(static_cast<size_t>(n) * 4);
    l.hist_stride = (l.nblocks + 3) & ~3;
    l.hist = off; off += up(static_cast<size_t>(kBins) * l.hist_stride * 4);
    l.heads = off; off += up(static_cast<size_t>(l.nblocks + 1) * 4);
    l.seg_start = off; off += up(static_cast<size_t>(n + 1) * 4);
    l.seg_pos = off; off += up(static_cast<size_t>(n) * 4);
    if (l.ng_max > 0) {
        l.tmp = off; off += up(static_cast<size_t>(n) * 8);
        l.gd_off = off; off += up(static_cast<size_t>(l.ntiles) * (l.ng_max + 1) * 4);
        l.gd_start = off; off += up(static_cast<size_t>(l.ng_max + 1) * 4);
        l.gd_ucount = off; off += up(static_cast<size_t>(l.ng_max) * 4);
    }
    l.total = off;
    return l;
}

// Group shift for the group dedup: the smallest s whose groups (key >> s) number at most
// ng_max; -1 when the group dedup is not used (ng_max 0) or the low key bits below a group
// would not fit the 32 bits of a composite.
int group_shift(int64_t key_bound, uint32_t ng_max) {
    if (ng_max == 0) return -1;
    const uint64_t top = static_cast<uint64_t>(key_bound - 1);
    int s = 0;
    while (s < 63 && (top >> s) + 1 > ng_max) ++s;
    return s <= 32 ? s : -1;
}

}  // namespace
}  // namespace me

using namespace me;

extern "C" int me_dedup_workspace_size(int64_t n, size_t *bytes) {
    ME_CHECK_ARG(bytes != nullptr, "bytes is null");
    ME_CHECK_ARG(n >= 0 && n < (int64_t{1} << 31), "n out of range");
    *bytes = dedup_layout(n).total;
    return ME_OK;
}

namespace me {
namespace {

// The segment plan both dedup paths leave for the sums: spos [n] (positions in sorted key
// order), seg_start [n + 1] (first index into spos of each unique key, then n), seg_pos [n]
// (first position of each unique key). Regions 256-byte aligned.
struct PlanLayout {
    size_t spos, seg_start, seg_pos, total;
};

PlanLayout plan_layout(int64_t n) {
    auto up = [](size_t x) { return (x + 255) & ~size_t{255}; };
    PlanLayout p{};
    size_t off = 0;
    p.spos = off; off += up(static_cast<size_t>(n) * 4);
    p.seg_start = off; off += up(static_cast<size_t>(n + 1) * 4);
    p.seg_pos = off; off += up(static_cast<size_t>(n) * 4);
    p.total = off;
    return p;
}

// The key half: unique keys, inverse, count and the segment plan (spos, seg_start, seg_pos).
int dedup_keys_run(const int64_t *keys, int64_t n, int64_t key_bound, int64_t *uniq, int64_t *inv,
                   int64_t *count, uint32_t *spos, uint32_t *seg_start, uint32_t *seg_pos,
                   uint8_t *ws, const DedupLayout &l, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(l.nblocks)), block(kThreads);
    const int shift = group_shift(key_bound, l.ng_max);
    if (shift >= 0) {
        // group dedup: per-tile grouping, per-group sort, the keys' emit
        const uint32_t ng = static_cast<uint32_t>((static_cast<uint64_t>(key_bound - 1) >> shift) + 1);
        uint64_t *tile_comp = reinterpret_cast<uint64_t *>(ws + l.keys_b);
        uint64_t *comp = tile_comp + n;
        uint64_t *tmp = reinterpret_cast<uint64_t *>(ws + l.tmp);
        uint32_t *off = reinterpret_cast<uint32_t *>(ws + l.gd_off);
        uint32_t *gstart = reinterpret_cast<uint32_t *>(ws + l.gd_start);
        uint32_t *ucount = reinterpret_cast<uint32_t *>(ws + l.gd_ucount);
        const uint64_t *k64 = reinterpret_cast<const uint64_t *>(keys);
        hipLaunchKernelGGL(gd_tile, dim3(l.ntiles), block, 0, s, k64, n, shift, ng, tile_comp, off);
        hipLaunchKernelGGL(gd_group, dim3(ng), block, 0, s, tile_comp, off, l.ntiles, ng, shift, n, comp,
                           tmp, gstart, ucount);
        hipLaunchKernelGGL(gd_emit, dim3(ng), block, 0, s, comp, gstart, ucount, ng, shift, uniq, inv, spos,
                           seg_start, seg_pos, count);
        return check_launch("me_dedup (keys, groups)");
    }
    // LSD radix sort of (key, position), 8 bits per pass, then the segments; the positions of
    // the last pass land in spos
    const int passes = (sort_bits(key_bound) + 7) / 8;
    uint64_t *kb[2] = {reinterpret_cast<uint64_t *>(ws + l.keys_b),
                       reinterpret_cast<uint64_t *>(ws + l.keys_b) + n};
    uint32_t *pb[2];
    pb[(passes - 1) & 1] = spos;
    pb[passes & 1] = reinterpret_cast<uint32_t *>(ws + l.pos_a);
    uint32_t *hist = reinterpret_cast<uint32_t *>(ws + l.hist);
    uint32_t *heads = reinterpret_cast<uint32_t *>(ws + l.heads);
    const uint64_t *kin = reinterpret_cast<const uint64_t *>(keys);
    const uint32_t *pin = nullptr;
    int cur = 0;
    for (int p = 0; p < passes; ++p) {
        const int sh = 8 * p;
        hipLaunchKernelGGL(rs_hist, grid, block, 0, s, kin, n, sh, hist, l.nblocks, l.hist_stride);
        hipLaunchKernelGGL(rs_scatter, grid, block, 0, s, kin, pin, kb[cur], pb[cur], n, sh, hist,
                           l.hist_stride);
        kin = kb[cur];
        pin = pb[cur];
        cur ^= 1;
    }
    const int st = check_launch("me_dedup (sort)");
    if (st != ME_OK) return st;
    hipLaunchKernelGGL(seg_count, grid, block, 0, s, kin, n, heads);
    hipLaunchKernelGGL(seg_write, grid, block, 0, s, kin, pin, n, heads, l.nblocks, uniq, inv,
                       seg_start, seg_pos, count);
    return check_launch("me_dedup (keys, segments)");
}

// The gradient half: each unique key's fp32 sum of its rows, from the plan.
int dedup_sums_run(const uint32_t *spos, const uint32_t *seg_start, const uint32_t *seg_pos,
                   const int64_t *count, int64_t n, const void *grads, int grad_dtype, int32_t dim,
                   float *gsum, hipStream_t s) {
    // four columns per thread when every row start is aligned for the vector loads and stores
    const size_t gsz = grad_dtype == ME_F32 ? 4 : 2;
    const bool vec = dim % 4 == 0 && reinterpret_cast<uintptr_t>(grads) % (4 * gsz) == 0 &&
                     reinterpret_cast<uintptr_t>(gsum) % 16 == 0;
    const int64_t threads = n * (vec ? dim / 4 : dim);
    ME_CHECK_ARG(threads < (int64_t{1} << 31), "n * dim = %lld too large for one call",
                 (long long)(n * dim));
    const dim3 sgrid(static_cast<unsigned>(ceil_div(threads, kThreads))), block(kThreads);
    const uint32_t d = static_cast<uint32_t>(dim), sp = static_cast<uint32_t>(n);
    if (grad_dtype == ME_F32) {
        const float *g = static_cast<const float *>(grads);
        if (vec)
            hipLaunchKernelGGL((seg_sum<float, 4>), sgrid, block, 0, s, g, d, spos, seg_start, seg_pos, count,
                               sp, gsum);
        else
            hipLaunchKernelGGL((seg_sum<float, 1>), sgrid, block, 0, s, g, d, spos, seg_start, seg_pos, count,
                               sp, gsum);
    } else {
        const uint16_t *g = static_cast<const uint16_t *>(grads);
        if (vec)
            hipLaunchKernelGGL((seg_sum<uint16_t, 4>), sgrid, block, 0, s, g, d, spos, seg_start, seg_pos,
                               count, sp, gsum);
        else
            hipLaunchKernelGGL((seg_sum<uint16_t, 1>), sgrid, block, 0, s, g, d, spos, seg_start, seg_pos,
                               count, sp, gsum);
    }
    return check_launch("me_dedup (sums)");
}

}  // namespace
}  // namespace me

extern "C" int me_dedup(const int64_t *keys, int64_t n, int64_t key_bound, const void *grads,
                        int grad_dtype, int32_t dim, int64_t *uniq, int64_t *inv, float *gsum,
                        int64_t *count, void *workspace, size_t workspace_size, void *stream) {
    ME_CHECK_ARG(n >= 0 && n < (int64_t{1} << 31), "n out of range");
    ME_CHECK_ARG(key_bound >= 1, "key_bound must be positive");
    ME_CHECK_ARG(count != nullptr, "count is null");
    ME_CHECK_ARG(grads == nullptr || grad_dtype == ME_F32 || grad_dtype == ME_BF16,
                 "grad dtype must be fp32 or bf16");
    ME_CHECK_ARG(grads == nullptr || dim >= 1, "dim must be positive");
    hipStream_t s = as_stream(stream);
    if (n == 0) {
        hipLaunchKernelGGL(write_zero_count, dim3(1), dim3(1), 0, s, count);
        return check_launch("me_dedup");
    }
    ME_CHECK_ARG(keys && uniq && inv, "null tensor pointer");
    ME_CHECK_ARG(grads == nullptr || gsum != nullptr, "gsum is null");
    const DedupLayout l = dedup_layout(n);
    if (workspace == nullptr || workspace_size < l.total) {
        set_error("me_dedup: workspace of %zu bytes needed, got %zu", l.total, workspace_size);
        return ME_ERR_WORKSPACE;
    }
    uint8_t *ws = static_cast<uint8_t *>(workspace);
    uint32_t *spos = reinterpret_cast<uint32_t *>(ws + l.pos_b);
    uint32_t *seg_start = reinterpret_cast<uint32_t *>(ws + l.seg_start);
    uint32_t *seg_pos = reinterpret_cast<uint32_t *>(ws + l.seg_pos);
    const int st = dedup_keys_run(keys, n, key_bound, uniq, inv, count, spos, seg_start, seg_pos, ws, l, s);
    if (st != ME_OK || grads == nullptr) return st;
    return dedup_sums_run(spos, seg_start, seg_pos, count, n, grads, grad_dtype, dim, gsum, s);
}

extern "C" int me_dedup_plan_size(int64_t n, size_t *bytes) {
    ME_CHECK_ARG(bytes != nullptr, "bytes is null");
    ME_CHECK_ARG(n >= 0 && n < (int64_t{1} << 31), "n out of range");
    *bytes = plan_layout(n).total;
    return ME_OK;
}

extern "C" int me_dedup_keys(const int64_t *keys, int64_t n, int64_t key_bound, int64_t *uniq,
                             int64_t *inv, int64_t *count, void *plan, size_t plan_size,
                             void *workspace, size_t workspace_size, void *stream) {
    ME_CHECK_ARG(n >= 0 && n < (int64_t{1} << 31), "n out of range");
    ME_CHECK_ARG(key_bound >= 1, "key_bound must be positive");
    ME_CHECK_ARG(count != nullptr, "count is null");
    hipStream_t s = as_stream(stream);
    if (n == 0) {
        hipLaunchKernelGGL(write_zero_count, dim3(1), dim3(1), 0, s, count);
        return check_launch("me_dedup_keys");
    }
    ME_CHECK_ARG(keys && uniq && inv, "null tensor pointer");
    const PlanLayout p = plan_layout(n);
    if (plan == nullptr || plan_size < p.total) {
        set_error("me_dedup_keys: plan of %zu bytes needed, got %zu", p.total, plan_size);
        return ME_ERR_WORKSPACE;
    }
    const DedupLayout l = dedup_layout(n);
    if (workspace == nullptr || workspace_size < l.total) {
        set_error("me_dedup_keys: workspace of %zu bytes needed, got %zu", l.total, workspace_size);
        return ME_ERR_WORKSPACE;
    }
    uint8_t *pl = static_cast<uint8_t *>(plan);
    return dedup_keys_run(keys, n, key_bound, uniq, inv, count, reinterpret_cast<uint32_t *>(pl + p.spos),
                          reinterpret_cast<uint32_t *>(pl + p.seg_start),
                          reinterpret_cast<uint32_t *>(pl + p.seg_pos), static_cast<uint8_t *>(workspace), l,
                          s);
}

// ---- table bounds of the unique keys --------------------------------------------------------
// The unique keys are concatenated-table keys (table offset + row), ascending: thread i finds the
// table of unique key i (the last offset <= key), writes its local row, and where the table
// changes between keys i - 1 and i it writes the first index of every table in between; the
// thread at the count closes the tables after the last key. info = [count, bound of table 0,
// ..., bound of table n_tables (= count)], the slices rows.py:125-129 hands each table.
namespace me {
namespace {
struct TableOffsets {
    int64_t off[ME_MAX_TABLES + 1];
};

__device__ __forceinline__ int table_of(int64_t key, const TableOffsets &t, int nt) {
    int lo = 0, hi = nt;  // off[lo] <= key < off[hi] for keys in range
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (t.off[mid] <= key) lo = mid; else hi = mid;
    }
    return lo;
}

__global__ __launch_bounds__(kThreads) void table_bounds_kernel(const int64_t *uniq, int64_t n,
                                                                const int64_t *count, TableOffsets t,
                                                                int nt, int64_t *local, int64_t *info) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t cnt = *count;
    if (i > cnt || i > n) return;
    const int tcur = i < cnt ? table_of(uniq[i], t, nt) : nt;
    const int tprev = i > 0 ? table_of(uniq[i - 1], t, nt) : -1;
    if (i < cnt) local[i] = uniq[i] - t.off[tcur];
    for (int k = tprev + 1; k <= tcur; ++k) info[1 + k] = i;
    if (i == 0) info[0] = cnt;
}
}  // namespace
}  // namespace me

extern "C" int me_dedup_table_bounds(const int64_t *uniq, int64_t n, const int64_t *count,
                                     const int64_t *table_offsets, int32_t n_tables, int64_t *local_rows,
                                     int64_t *info, void *stream) {
    ME_CHECK_ARG(n >= 0 && n < (int64_t{1} << 31), "n out of range");
    ME_CHECK_ARG(n_tables >= 1 && n_tables <= ME_MAX_TABLES, "n_tables must be in [1, %d]", ME_MAX_TABLES);
    ME_CHECK_ARG(count && table_offsets && info && (n == 0 || (uniq && local_rows)), "null pointer");
    TableOffsets t{};
    for (int k = 0; k <= n_tables; ++k) {
        t.off[k] = table_offsets[k];
        ME_CHECK_ARG(k == 0 || t.off[k] >= t.off[k - 1], "table offsets must be ascending");
    }
    ME_CHECK_ARG(t.off[0] == 0, "the first table offset must be 0");
    const dim3 grid(static_cast<unsigned>(ceil_div(n + 1, kThreads)));
    hipLaunchKernelGGL(table_bounds_kernel, grid, dim3(kThreads), 0, as_stream(stream), uniq, n, count, t,
                       n_tables, local_rows, info);
    return check_launch("me_dedup_table_bounds");
}

// ---- the key half from per-table row ids ------------------------------------------------------
namespace me {
namespace {
__global__ __launch_bounds__(kThreads) void td_keys(const TdArgs a, int64_t *keys) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t total = static_cast<int64_t>(a.n) * a.nt;
    if (i >= total) return;
    const int64_t t = i / a.nt;
    const int k = static_cast<int>(i - t * a.nt);
    const int64_t v = a.idx[static_cast<int64_t>(k) * a.stride + t];
    const int64_t rmax = a.rows[k] - 1;
    keys[i] = a.off[k] + (v < 0 ? 0 : (v > rmax ? rmax : v));
}

__global__ void td_empty_info(int64_t *info, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) info[i] = 0;
}

struct TdLayout {
    bool fast;  // the two-launch table path (else: keys, then the generic key half + bounds)
    size_t srow, tmp_a, tmp_b, slot, gstart, gsize, ucount;  // fast path
    size_t keys, inv;                                   // generic path, then its DedupLayout
    DedupLayout dl;
    size_t total;
};

// Fills the table description of a and returns the workspace layout for it.
int td_setup(TdArgs &a, const int64_t *idx, int64_t stride, int64_t n, int32_t nt,
             const int64_t *table_rows, TdLayout *out) {
    ME_CHECK_ARG(n >= 0 && nt >= 1 && nt <= ME_MAX_TABLES, "bad n / n_tables");
    ME_CHECK_ARG(n * nt < (int64_t{1} << 31), "n * n_tables = %lld too large", (long long)(n * nt));
    ME_CHECK_ARG(table_rows != nullptr, "table_rows is null");
    ME_CHECK_ARG(stride >= n, "idx_table_stride %lld < n %lld", (long long)stride, (long long)n);
    a.idx = idx;
    a.stride = stride;
    a.n = static_cast<uint32_t>(n);
    a.nt = nt;
    bool fast = n <= kTdMaxN;
    const int64_t target = std::max<int64_t>(1, ceil_div(n, kTdPartTarget));
    int64_t off = 0;
    uint32_t ng = 0;
    for (int k = 0; k < nt; ++k) {
        ME_CHECK_ARG(table_rows[k] >= 1, "table %d has %lld rows", k, (long long)table_rows[k]);
        a.rows[k] = table_rows[k];
        a.off[k] = off;
        off += table_rows[k];
        fast = fast && table_rows[k] <= (int64_t{1} << 32);
        a.shift[k] = td_shift(table_rows[k], target);
        a.gbase[k] = ng;
        ng += static_cast<uint32_t>(((table_rows[k] - 1) >> a.shift[k]) + 1);
    }
    a.gbase[nt] = ng;
    a.ngroups = ng;
    const int64_t N = n * nt;
    auto up = [](size_t x) { return (x + 255) & ~size_t{255}; };
    TdLayout l{};
    l.fast = fast;
    size_t o = 0;
    if (fast) {
        l.srow = o; o += up(static_cast<size_t>(N) * 4);
        l.tmp_a = o; o += up(static_cast<size_t>(N) * 8);
        l.tmp_b = o; o += up(static_cast<size_t>(N) * 8);
        l.slot = o; o += up(static_cast<size_t>(ng) * kTdCap * 8);
        l.gstart = o; o += up(static_cast<size_t>(ng) * 4);
        l.gsize = o; o += up(static_cast<size_t>(ng) * 4);
        l.ucount = o; o += up(static_cast<size_t>(ng) * 4);
    } else {
        l.keys = o; o += up(static_cast<size_t>(N) * 8);
        l.inv = o; o += up(static_cast<size_t>(N) * 8);  // the inverse when the caller wants none
        l.dl = dedup_layout(N);
        o += l.dl.total;
    }
    l.total = o;
    *out = l;
    return ME_OK;
}
}  // namespace
}  // namespace me

extern "C" int me_dedup_tables_workspace_size(int64_t n, int32_t n_tables, const int64_t *table_rows,
                                              size_t *bytes) {
    ME_CHECK_ARG(bytes != nullptr, "bytes is null");
    TdArgs a{};
    TdLayout l{};
    const int st = td_setup(a, nullptr, n, n, n_tables, table_rows, &l);
    if (st != ME_OK) return st;
    *bytes = l.total;
    return ME_OK;
}

extern "C" int me_dedup_tables(const int64_t *idx, int64_t idx_table_stride, int64_t n, int32_t n_tables,
                               const int64_t *table_rows, int64_t *uniq, int64_t *local_rows, int64_t *inv,
                               int64_t *info, void *plan, size_t plan_size, void *workspace,
                               size_t workspace_size, void *stream) {
    TdArgs a{};
    TdLayout l{};
    const int st = td_setup(a, idx, idx_table_stride, n, n_tables, table_rows, &l);
    if (st != ME_OK) return st;
    ME_CHECK_ARG(info != nullptr, "info is null");
    hipStream_t s = as_stream(stream);
    if (n == 0) {
        hipLaunchKernelGGL(td_empty_info, dim3(1), dim3(64), 0, s, info, n_tables + 2);
        return check_launch("me_dedup_tables");
    }
    ME_CHECK_ARG(idx && uniq && local_rows, "null tensor pointer");
    const int64_t N = n * n_tables;
    const PlanLayout p = plan_layout(N);
    if (plan == nullptr || plan_size < p.total) {
        set_error("me_dedup_tables: plan of %zu bytes needed, got %zu", p.total, plan_size);
        return ME_ERR_WORKSPACE;
    }
    if (workspace == nullptr || workspace_size < l.total) {
        set_error("me_dedup_tables: workspace of %zu bytes needed, got %zu", l.total, workspace_size);
        return ME_ERR_WORKSPACE;
    }
    uint8_t *pl = static_cast<uint8_t *>(plan);
    uint8_t *ws = static_cast<uint8_t *>(workspace);
    a.spos = reinterpret_cast<uint32_t *>(pl + p.spos);
    a.seg_start = reinterpret_cast<uint32_t *>(pl + p.seg_start);
    a.seg_pos = reinterpret_cast<uint32_t *>(pl + p.seg_pos);
    a.uniq = uniq;
    a.local = local_rows;
    a.inv = inv;
    a.info = info;
    if (l.fast) {
        a.srow = reinterpret_cast<uint32_t *>(ws + l.srow);
        a.tmp_a = reinterpret_cast<uint64_t *>(ws + l.tmp_a);
        a.tmp_b = reinterpret_cast<uint64_t *>(ws + l.tmp_b);
        a.slot = reinterpret_cast<uint64_t *>(ws + l.slot);
        a.gstart = reinterpret_cast<uint32_t *>(ws + l.gstart);
        a.gsize = reinterpret_cast<uint32_t *>(ws + l.gsize);
        a.ucount = reinterpret_cast<uint32_t *>(ws + l.ucount);
        const bool vec2 = reinterpret_cast<uintptr_t>(idx) % 16 == 0 && idx_table_stride % 2 == 0 && n % 2 == 0;
        const int rounds = static_cast<int>(ceil_div(n, 2 * kThreads));
        const dim3 grid(a.ngroups), block(kThreads);
#define ME_TD_PART(R)                                                                   \
    if (rounds <= R) {                                                                  \
        if (vec2) hipLaunchKernelGGL((td_part<R, true>), grid, block, 0, s, a);         \
        else hipLaunchKernelGGL((td_part<R, false>), grid, block, 0, s, a);             \
    } else
        ME_TD_PART(1) ME_TD_PART(2) ME_TD_PART(4) ME_TD_PART(8) ME_TD_PART(16) {}
#undef ME_TD_PART
        hipLaunchKernelGGL(td_emit, dim3(a.ngroups), dim3(kThreads), 0, s, a);
        return check_launch("me_dedup_tables");
    }
    // more tokens than the table path takes: the keys, the generic key half, the bounds
    int64_t *keys = reinterpret_cast<int64_t *>(ws + l.keys);
    hipLaunchKernelGGL(td_keys, dim3(static_cast<unsigned>(ceil_div(N, kThreads))), dim3(kThreads), 0, s, a,
                       keys);
    const int64_t key_bound = a.off[n_tables - 1] + a.rows[n_tables - 1];
    int64_t *inv_out = inv != nullptr ? inv : reinterpret_cast<int64_t *>(ws + l.inv);
    const int st2 = dedup_keys_run(keys, N, key_bound, uniq, inv_out, info, a.spos, a.seg_start, a.seg_pos,
                                   ws + (l.inv + ((static_cast<size_t>(N) * 8 + 255) & ~size_t{255})), l.dl,
                                   s);
    if (st2 != ME_OK) return st2;
    TableOffsets t{};
    for (int k = 0; k < n_tables; ++k) t.off[k] = a.off[k];
    t.off[n_tables] = key_bound;
    hipLaunchKernelGGL(table_bounds_kernel, dim3(static_cast<unsigned>(ceil_div(N + 1, kThreads))),
                       dim3(kThreads), 0, s, uniq, N, info, t, n_tables, local_rows, info);
    return check_launch("me_dedup_tables (generic)");
}

extern "C" int me_dedup_sums(const void *plan, size_t plan_size, int64_t n, const int64_t *count,
                             const void *grads, int grad_dtype, int32_t dim, float *gsum, void *stream) {
    ME_CHECK_ARG(n >= 0 && n < (int64_t{1} << 31), "n out of range");
    ME_CHECK_ARG(grad_dtype == ME_F32 || grad_dtype == ME_BF16, "grad dtype must be fp32 or bf16");
    ME_CHECK_ARG(dim >= 1, "dim must be positive");
    if (n == 0) return ME_OK;
    ME_CHECK_ARG(count && grads && gsum, "null tensor pointer");
    const PlanLayout p = plan_layout(n);
    if (plan == nullptr || plan_size < p.total) {
        set_error("me_dedup_sums: plan of %zu bytes needed, got %zu", p.total, plan_size);
        return ME_ERR_WORKSPACE;
    }
    const uint8_t *pl = static_cast<const uint8_t *>(plan);
    return dedup_sums_run(reinterpret_cast<const uint32_t *>(pl + p.spos),
                          reinterpret_cast<const uint32_t *>(pl + p.seg_start),
                          reinterpret_cast<const uint32_t *>(pl + p.seg_pos), count, n, grads, grad_dtype,
                          dim, gsum, as_stream(stream));
}

extern "C" int me_sumsq(const float *x, int64_t n, float *out, int accumulate, void *workspace,
                        size_t workspace_size, void *stream) {
    ME_CHECK_ARG(out != nullptr, "out is null");
    ME_CHECK_ARG(n >= 0, "negative n");
    ME_CHECK_ARG(x != nullptr || n == 0, "x is null");
    if (workspace == nullptr || workspace_size < kSumBlocks * sizeof(float)) {
        set_error("me_sumsq: workspace of %zu bytes needed, got %zu", kSumBlocks * sizeof(float),
                  workspace_size);
        return ME_ERR_WORKSPACE;
    }
    float *partial = static_cast<float *>(workspace);
    hipStream_t s = as_stream(stream);
    hipLaunchKernelGGL(sumsq_partial, dim3(kSumBlocks), dim3(kSumThreads), 0, s, x, n, partial);
    hipLaunchKernelGGL(sumsq_final, dim3(1), dim3(kSumBlocks), 0, s, partial, out, accumulate);
    return check_launch("me_sumsq");
}

extern "C" int me_clip_scale(void *x, int dtype, int64_t n, const float *sumsq, double max_norm,
                             void *stream) {
    ME_CHECK_ARG(n >= 0, "negative n");
    ME_CHECK_ARG(x != nullptr || n == 0, "x is null");
    ME_CHECK_ARG(sumsq != nullptr, "sumsq is null");
    ME_CHECK_ARG(dtype == ME_F32 || dtype == ME_BF16, "x must be fp32 or bf16");
    ME_CHECK_ARG(reinterpret_cast<uintptr_t>(x) % 16 == 0, "x must be 16-byte aligned");
    ME_CHECK_ARG(max_norm > 0.0, "max_norm must be positive");
    if (n == 0) return ME_OK;
    const int per = dtype == ME_BF16 ? 8 : 4;
    const int64_t blocks = std::min<int64_t>(std::max<int64_t>(ceil_div(n / per, kClipThreads), 1), 2048);
    hipStream_t s = as_stream(stream);
    const float mn = static_cast<float>(max_norm);
    if (dtype == ME_BF16)
        hipLaunchKernelGGL(clip_scale<true>, dim3(static_cast<unsigned>(blocks)), dim3(kClipThreads), 0,
                           s, x, n, sumsq, mn);
    else
        hipLaunchKernelGGL(clip_scale<false>, dim3(static_cast<unsigned>(blocks)), dim3(kClipThreads), 0,
                           s, x, n, sumsq, mn);
    return check_launch("me_clip_scale");
}

template <int C, bool PB, bool RW, bool GB>
void launch_adam_vec_k(int lpr, dim3 grid, hipStream_t s, const AdamArgs &a) {
    switch (lpr) {
        case 1: hipLaunchKernelGGL((adam_rows_vec<1, C, PB, RW, GB>), grid, dim3(kThreads), 0, s, a); break;
        case 2: hipLaunchKernelGGL((adam_rows_vec<2, C, PB, RW, GB>), grid, dim3(kThreads), 0, s, a); break;
        case 4: hipLaunchKernelGGL((adam_rows_vec<4, C, PB, RW, GB>), grid, dim3(kThreads), 0, s, a); break;
        case 8: hipLaunchKernelGGL((adam_rows_vec<8, C, PB, RW, GB>), grid, dim3(kThreads), 0, s, a); break;
        case 16: hipLaunchKernelGGL((adam_rows_vec<16, C, PB, RW, GB>), grid, dim3(kThreads), 0, s, a); break;
        case 32: hipLaunchKernelGGL((adam_rows_vec<32, C, PB, RW, GB>), grid, dim3(kThreads), 0, s, a); break;
        default: hipLaunchKernelGGL((adam_rows_vec<64, C, PB, RW, GB>), grid, dim3(kThreads), 0, s, a); break;
    }
}

template <int C, bool GB>
void launch_adam_vec_g(int lpr, bool pb, bool rw, dim3 grid, hipStream_t s, const AdamArgs &a) {
    if (pb)
        rw ? launch_adam_vec_k<C, true, true, GB>(lpr, grid, s, a) : launch_adam_vec_k<C, true, false, GB>(lpr, grid, s, a);
    else
        rw ? launch_adam_vec_k<C, false, true, GB>(lpr, grid, s, a) : launch_adam_vec_k<C, false, false, GB>(lpr, grid, s, a);
}

template <int C>
void launch_adam_vec(int lpr, bool pb, bool rw, bool gb, dim3 grid, hipStream_t s, const AdamArgs &a) {
    gb ? launch_adam_vec_g<C, true>(lpr, pb, rw, grid, s, a) : launch_adam_vec_g<C, false>(lpr, pb, rw, grid, s, a);
}

template <bool GB>
void launch_adam_wide(bool pb, bool rw, dim3 grid, hipStream_t s, const AdamArgs &a) {
    if (pb && rw)
        hipLaunchKernelGGL((adam_rows_wide<8, true, true, GB>), grid, dim3(kThreads), 0, s, a);
    else if (pb)
        hipLaunchKernelGGL((adam_rows_wide<8, true, false, GB>), grid, dim3(kThreads), 0, s, a);
    else if (rw)
        hipLaunchKernelGGL((adam_rows_wide<8, false, true, GB>), grid, dim3(kThreads), 0, s, a);
    else
        hipLaunchKernelGGL((adam_rows_wide<8, false, false, GB>), grid, dim3(kThreads), 0, s, a);
}

extern "C" int me_sparse_adam(int32_t n_tables, void *const *params, void *const *exp_avgs,
                              void *const *exp_avg_sqs, const int64_t *const *rows,
                              const void *const *grads, int grad_dtype, const int64_t *n_rows,
                              const int64_t *steps, const int32_t *stream_ids, int32_t dim,
                              int param_dtype, int rowwise, int sq_dtype, int lazy, double lr,
                              double beta1, double beta2, double eps, double weight_decay,
                              int stochastic_rounding, uint64_t seed, void *stream) {
    ME_CHECK_ARG(n_tables >= 1 && n_tables <= 65536, "n_tables must be in [1, 65536]");
    ME_CHECK_ARG(params && exp_avgs && exp_avg_sqs && rows && grads && n_rows && steps && stream_ids,
                 "null argument array");
    ME_CHECK_ARG(param_dtype == ME_BF16 || param_dtype == ME_F32, "param dtype must be bf16/fp32");
    ME_CHECK_ARG(grad_dtype == ME_BF16 || grad_dtype == ME_F32, "grad dtype must be bf16/fp32");
    ME_CHECK_ARG(dim >= 1, "dim must be positive");
    ME_CHECK_ARG(rowwise || sq_dtype == ME_BF16 || sq_dtype == ME_F32, "bad second-moment dtype");
    AdamArgs a{};
    a.dim = dim;
    a.param_bf16 = param_dtype == ME_BF16;
    a.rowwise = rowwise != 0;
    a.sq_bf16 = !rowwise && sq_dtype == ME_BF16;
    a.grad_bf16 = grad_dtype == ME_BF16;
    a.sr = stochastic_rounding != 0;
    a.lazy = lazy != 0;
    a.seed = seed;
    a.has_decay = weight_decay != 0.0;
    a.decay = static_cast<float>(1.0 - lr * weight_decay);
    a.beta1 = static_cast<float>(beta1);
    a.one_minus_beta1 = static_cast<float>(1.0 - beta1);
    a.beta2 = static_cast<float>(beta2);
    a.one_minus_beta2 = static_cast<float>(1.0 - beta2);
    a.eps = static_cast<float>(eps);
    for (int k = 0; k < n_tables; ++k) {
        ME_CHECK_ARG(n_rows[k] >= 0, "table %d: negative row count", k);
        ME_CHECK_ARG(steps[k] >= 1, "table %d: step must be >= 1", k);
        ME_CHECK_ARG(n_rows[k] == 0 || (params[k] && exp_avgs[k] && exp_avg_sqs[k] && rows[k] && grads[k]),
                     "table %d: null tensor pointer", k);
        ME_CHECK_ARG(stream_ids[k] >= 0 && stream_ids[k] < 65536, "table %d: stream id out of range", k);
    }
    for (int k0 = 0; k0 < n_tables; k0 += kAdamTables) {
        const int nk = min(kAdamTables, n_tables - k0);
        int64_t total = 0;
        for (int q = 0; q < nk; ++q) {
            const int k = k0 + q;
            AdamTable &t = a.t[q];
            t.param = static_cast<uint8_t *>(params[k]);
            t.exp_avg = static_cast<uint8_t *>(exp_avgs[k]);
            t.exp_avg_sq = static_cast<uint8_t *>(exp_avg_sqs[k]);
            t.rows = rows[k];
            t.grads = static_cast<const uint8_t *>(grads[k]);
            t.n = n_rows[k];
            t.first = total;
            const double step = static_cast<double>(steps[k]);
            const double bc1 = 1.0 - std::pow(beta1, step), bc2 = 1.0 - std::pow(beta2, step);
            t.neg_lr_bc1 = static_cast<float>(-lr / bc1);
            t.sqrt_bc2 = static_cast<float>(std::sqrt(bc2));
            t.step = static_cast<uint32_t>(steps[k]);
            t.stream_id = static_cast<uint32_t>(stream_ids[k]);
            total += n_rows[k];
        }
        a.n_tables = nk;
        a.total = total;
        if (total == 0) continue;
        // vector paths: dim = C * lanes-per-row (C = 8 columns per lane, else 4) with
        // lanes-per-row a power of two <= 64, and every row start aligned for C-element loads
        auto fits = [&](int c) {
            const int lpr = dim % c == 0 ? dim / c : 0;
            if (lpr < 1 || lpr > 64 || (lpr & (lpr - 1)) != 0) return 0;
            const uintptr_t pal = a.param_bf16 ? 2 * c : 16, val = a.rowwise ? 4 : (a.sq_bf16 ? 2 * c : 16);
            for (int q = 0; q < nk; ++q) {
                const AdamTable &t = a.t[q];
                if (reinterpret_cast<uintptr_t>(t.param) % pal != 0 ||
                    reinterpret_cast<uintptr_t>(t.exp_avg) % pal != 0 ||
                    reinterpret_cast<uintptr_t>(t.exp_avg_sq) % val != 0 ||
                    reinterpret_cast<uintptr_t>(t.grads) % 16 != 0)
                    return 0;
            }
            return lpr;
        };
        hipStream_t s = as_stream(stream);
        const int lpr8 = fits(8), lpr4 = lpr8 ? 0 : fits(4);
        // rows of whole 64-lane blocks of 8 columns (wider than one pass of adam_rows_vec)
        const bool wide = !lpr8 && !lpr4 && dim % 512 == 0 &&
                          [&] {
                              const uintptr_t pal = 16, val = a.rowwise ? 4 : 16;
                              for (int q = 0; q < nk; ++q) {
                                  const AdamTable &t = a.t[q];
                                  if (reinterpret_cast<uintptr_t>(t.param) % pal != 0 ||
                                      reinterpret_cast<uintptr_t>(t.exp_avg) % pal != 0 ||
                                      reinterpret_cast<uintptr_t>(t.exp_avg_sq) % val != 0 ||
                                      reinterpret_cast<uintptr_t>(t.grads) % 16 != 0)
                                      return false;
                              }
                              return true;
                          }();
        if (wide) {
            const dim3 grid(static_cast<unsigned>(ceil_div(total, kThreads / 64)));
            if (a.grad_bf16)
                launch_adam_wide<true>(a.param_bf16 != 0, a.rowwise != 0, grid, s, a);
            else
                launch_adam_wide<false>(a.param_bf16 != 0, a.rowwise != 0, grid, s, a);
        } else if (lpr8 || lpr4) {
            const int lpr = lpr8 ? lpr8 : lpr4;
            const int64_t per_block = (64 / lpr) * (kThreads / 64);
            const dim3 grid(static_cast<unsigned>(ceil_div(total, per_block)));
            if (lpr8)
                launch_adam_vec<8>(lpr, a.param_bf16 != 0, a.rowwise != 0, a.grad_bf16 != 0, grid, s, a);
            else
                launch_adam_vec<4>(lpr, a.param_bf16 != 0, a.rowwise != 0, a.grad_bf16 != 0, grid, s, a);
        } else {
            const dim3 grid(static_cast<unsigned>(ceil_div(total, kThreads / 64)));
            hipLaunchKernelGGL(adam_rows, grid, dim3(kThreads), 0, s, a);
        }
        const int st = check_launch("me_sparse_adam");
        if (st != ME_OK) return st;
    }
    return ME_OK;
}

extern "C" int me_stochastic_bf16(const float *x, int64_t n, uint16_t *out, uint64_t seed,
                                  uint32_t step, uint32_t stream_id, void *stream) {
    ME_CHECK_ARG(n >= 0, "negative n");
    ME_CHECK_ARG((x != nullptr && out != nullptr) || n == 0, "null tensor pointer");
    ME_CHECK_ARG(stream_id < 65536, "stream id out of range");
    if (n == 0) return ME_OK;
    hipLaunchKernelGGL(sr_convert, dim3(static_cast<unsigned>(ceil_div(n, kThreads))), dim3(kThreads), 0,
                       as_stream(stream), x, n, out, seed, step, stream_id);
    return check_launch("me_stochastic_bf16");
}
