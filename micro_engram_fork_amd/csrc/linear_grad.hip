// Gradients of the engram's key / value Linear layers on gfx950: the GEMMs autograd runs for
// the two nn.Linear calls of the reference's forward (micro_engram/module.py:245, 254), from the
// gradients gK, gV [N, d] of their outputs that me_gate_backward leaves:
//
//   grad_mem [N, M] = gK . W_K + gV . W_V        (W_K, W_V [d, M]: nn.Linear weights [out, in])
//   grad_W_K [d, M] = gK^T . mem,  grad_W_V [d, M] = gV^T . mem        (mem [N, M])
//
// bf16 operands, fp32 accumulation over the whole reduction (both products of grad_mem in one
// accumulator), one round-to-nearest-even to bf16 per output element.
//
// One kernel for both: C [R, S] = sum over k of A(r, k) B(s, k), on 256 (R) x TS (S) output
// tiles of a 256-thread workgroup, four waves of 128 x TS/2 each, v_mfma_f32_16x16x32_bf16.
// The K loop is the one of the gate's projection kernel: 64-wide k-slabs (128 bytes of bf16)
// streamed through five 32 KiB LDS units by buffer_load ... lds (no VGPR staging), A of slab s
// in unit 2s % 5 and B in (2s + 1) % 5, one workgroup barrier per slab. What differs is the
// operands' layout in HBM:
//   k-contiguous  [rows][K] (gK for grad_mem): a unit holds 256 rows x 128 bytes, the eight
//                 16-byte chunks of a row XOR-swizzled by ((row >> 1) & 7); a fragment is one
//                 ds_read_b128 per lane (row l & 15, k chunk l >> 4).
//   row-contiguous [K][cols] (W for grad_mem; gK and mem for grad_W, whose reduction runs over
//                 tokens): a unit holds 64 k-rows x 512 bytes (256 columns), the 32 chunks of a
//                 k-row XOR-swizzled by 2 ((kr & 3) | ((kr >> 1) & 4)). A fragment is two
//                 ds_read_b64_tr_b16: each 16-lane group reads a 4 k x 16 column block (lane i
//                 addresses k-row i / 4, columns 4 (i % 4) .. +3) and lane i receives column i's
//                 four k values -- the MFMA operand layout, with no transpose through VGPRs
//                 or HBM. The swizzle puts the 8 k-rows x 2 chunks that the 32 lanes of one LDS
//                 cycle read on 16 distinct 16-byte bank groups.
// The tiles of grad_mem are 256 tokens x 192 memory columns (the Gemma-scale 8192 x 1536 output
// is 256 tiles: one per CU), those of grad_W 256 x 256 (two 5376 x 1536 outputs: 252 tiles).
// Workgroup ids are remapped so that each XCD's CUs take consecutive tiles, which share rows
// of A in that XCD's L2. Epilogue: each wave stages its bf16 tile in LDS and writes whole
// 16-byte row chunks.
#include "me_common.h"

#include <algorithm>
#include <type_traits>

namespace me {
namespace {

constexpr int kThreads = 256;
constexpr int kUnit = 32768;                  // one operand of one slab
constexpr int kUnits = 5;
constexpr int kRingBytes = kUnits * kUnit;    // 160 KiB
constexpr int kSlabK = 64;                    // k values per slab
constexpr int kSlabBytes = kSlabK * 2;        // 128 bytes of a k-contiguous row
constexpr int kTileR = 256;                   // output rows per tile
constexpr int kRcPitch = 512;                 // bytes of a k-row of a row-contiguous unit
constexpr int kDma = 8;                       // 1 KiB loads per wave per operand per slab
constexpr int kXcds = 8;
constexpr uint32_t kBufferConfig = 0x00020000u;  // raw buffer descriptor word 3 (gfx9 family)
constexpr uint32_t kOff = 0xffffffffu;        // a load offset past every buffer: reads zeros

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef int int32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

struct Operand {
    const void *base;
    uint32_t bytes;  // buffer size (under 2^31)
    int64_t ld;      // elements from one row to the next in HBM
};

// Problem p (of `problems`) writes C_p [R, S] from the sum over segments q (of `ksegs`) of
// A_{p+q} B_{p+q} (grad_mem: one problem, two segments; grad_W: up to two problems, one segment).
struct LgArgs {
    Operand a[2], b[2];
    uint16_t *c[2];
    int64_t ldc;
    int64_t R, S, K;  // output rows, output columns, reduction length of one segment
    int ksegs, problems, n_rt, n_st, total, per_xcd;
};

__device__ __forceinline__ int32x4 buffer_rsrc(const void *base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    int32x4 r;
    r.x = static_cast<int>(static_cast<uint32_t>(a));
    r.y = static_cast<int>(static_cast<uint32_t>(a >> 32) & 0xffffu);  // stride 0
    r.z = static_cast<int>(bytes);
    r.w = static_cast<int>(kBufferConfig);
    return r;
}

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) uint8_t *)p));
}

// One wave moves 64 x 16 bytes: lane l's chunk at byte voffset (+ soffset) of the buffer lands at
// LDS address lds_base + 16 l. The range check looks at voffset: a voffset at or past the buffer's
// size reads zeros. Counted by vmcnt; the caller waits explicitly.
__device__ __forceinline__ void dma16(const int32x4 &rsrc, uint32_t lds_base, uint32_t voffset,
                                      uint32_t soffset) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(lds_base), "v"(voffset), "s"(rsrc), "s"(soffset)
                 : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

__device__ __forceinline__ float acc_read(const floatx16 &t, int e) {
    float v;
    asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(t[e]));
    return v;
}

// XOR swizzle (in 16-byte chunks) of k-row kr of a row-contiguous unit
__device__ __forceinline__ int rc_swizzle(int kr) { return 4 * (kr & 3); }

// A 32x32x16 MFMA operand holds, in lane l, the 8 k values 16 ks + 8 (l >> 5) .. + 7 of row /
// column l & 31 of a 32-wide subtile.
//
// Row-contiguous unit: two transpose reads per fragment. 16-lane group g takes columns
// 16 (g & 1) .. + 15 of the subtile and k-rows 16 ks + 8 (g >> 1) + 4 half .. + 3; its lane i
// addresses k-row (i >> 2) of those four at columns 4 (i & 3) .. + 3. The swizzle 4 (kr & 3)
// of a k-row depends on i only, so k-step and half are constant byte offsets (8192 and 2048).
// The 32 lanes of one LDS cycle read 4 k-rows x 4 chunks, on 16 distinct 16-byte bank groups.
__device__ __forceinline__ uint32_t rc_lane_off(int col0, int lane) {
    const int i = lane & 15, g = lane >> 4;
    const int c = col0 + 16 * (g & 1) + 4 * (i & 3);
    const int kr = 8 * (g >> 1) + (i >> 2);
    return static_cast<uint32_t>(kr * kRcPitch + (((c >> 3) ^ rc_swizzle(kr)) << 4) + (c & 7) * 2);
}

__device__ __forceinline__ bf16x8 rc_frag(const uint8_t *unit, int ks, uint32_t off) {
    const auto *p = (const __attribute__((address_space(3))) uint8_t *)(unit + off) + ks * 16 * kRcPitch;
    const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4 *)(p));
    const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4 *)(p + 4 * kRcPitch));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// k-contiguous unit: one ds_read_b128 of row `row` at logical chunk 2 ks + (lane >> 5).
__device__ __forceinline__ bf16x8 kc_frag(const uint8_t *unit, int ks, int row, int lane) {
    const int c = ((2 * ks + (lane >> 5)) ^ ((row >> 1) & 7)) << 4;
    return *reinterpret_cast<const bf16x8 *>(unit + row * kSlabBytes + c);
}

template <bool A_KC, int TS>
__global__ __launch_bounds__(kThreads, 1) void linear_grad_kernel(const LgArgs a) {
    constexpr int kWS = TS / 2;             // output columns per wave
    constexpr int kSubS = kWS / 32;         // 32-column subtiles per wave (MFMA src0)
    constexpr int kSubR = 128 / 32;         // 32-row subtiles per wave (MFMA src1)
    constexpr int kParts = kSubS + kSubR;   // fragments per k-step
    constexpr int kMfma = kSubS * kSubR;    // MFMAs per k-step (4 k-steps per slab)
    constexpr int kPre = 4;                 // last k-step's MFMAs before the slab's barrier
    static_assert(kParts <= kMfma && 2 * kDma <= 4 * kMfma && kMfma - kPre >= kParts, "schedule fits");
    static_assert(TS % 64 == 0 && TS <= kRcPitch / 2, "a slab of B fits a unit");
    constexpr int kPitch = kWS * 2 + 16;    // staged output row (bytes)
    static_assert(4 * 128 * kPitch <= kRingBytes, "the epilogue stage fits the ring");
    __shared__ __attribute__((aligned(16))) uint8_t ring[kRingBytes];

    // ---- tile: consecutive logical tiles (same A rows, successive column tiles) on one XCD
    const int bid = blockIdx.x;
    const int logical = (bid % kXcds) * a.per_xcd + bid / kXcds;
    if (logical >= a.total) return;
    const int per_problem = a.n_rt * a.n_st;
    const int prob = logical / per_problem;
    const int rem = logical - prob * per_problem;
    const int rt = rem / a.n_st, st = rem - (rem / a.n_st) * a.n_st;
    const int64_t r0 = static_cast<int64_t>(rt) * kTileR;
    const int64_t s0 = static_cast<int64_t>(st) * TS;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave >> 1, ws = wave & 1;
    const int spq = static_cast<int>(ceil_div(a.K, kSlabK));  // slabs per segment
    const int slabs = spq * a.ksegs;

    // the operands of segment 0 and segment 1 (problem `prob` has one segment: both the same)
    const int o1 = min(prob + 1, 1);
    const int32x4 rsrc_a0 = buffer_rsrc(a.a[prob].base, a.a[prob].bytes);
    const int32x4 rsrc_b0 = buffer_rsrc(a.b[prob].base, a.b[prob].bytes);
    const int32x4 rsrc_a1 = buffer_rsrc(a.a[o1].base, a.a[o1].bytes);
    const int32x4 rsrc_b1 = buffer_rsrc(a.b[o1].base, a.b[o1].bytes);

    // ---- per-lane load offsets, fixed for the K loop.
    // k-contiguous A: load i of a wave fills rows 8 (8 wave + i) + [0, 8); lane l writes row
    // + l / 8 at physical chunk l % 8 (logical chunk (l % 8) ^ ((row >> 1) & 7)); the slab's
    // byte offset in the row goes in soffset (rows are whole slabs: K % 64 == 0).
    // row-contiguous: load i fills k-rows 2 (8 wave + i) + [0, 2); lane l writes k-row
    // + l / 32 at physical chunk l % 32 (logical chunk q = (l % 32) ^ swizzle), columns
    // tile0 + 8 q .. + 7 (past the tile or the matrix: reads zeros).
    const int hi = lane >> 5;
    uint32_t offa[kDma], offb[kDma];
    const int64_t lda = a.a[prob].ld, ldb = a.b[prob].ld;
#pragma unroll
    for (int i = 0; i < kDma; ++i) {
        if constexpr (A_KC) {
            const int row = (wave * kDma + i) * 8 + (lane >> 3);
            const uint32_t ch = static_cast<uint32_t>((lane & 7) ^ ((row >> 1) & 7)) * 16u;
            offa[i] = r0 + row < a.R ? static_cast<uint32_t>((r0 + row) * lda * 2) + ch : kOff;
        } else {
            const int kr = 2 * (wave * kDma + i) + hi;
            const int q = (lane & 31) ^ rc_swizzle(kr);
            const int64_t col = r0 + 8 * q;
            offa[i] = 8 * q < kTileR && col < a.R ? static_cast<uint32_t>((kr * lda + col) * 2) : kOff;
        }
        const int kr = 2 * (wave * kDma + i) + hi;
        const int q = (lane & 31) ^ rc_swizzle(kr);
        const int64_t col = s0 + 8 * q;
        offb[i] = 8 * q < TS && col < a.S ? static_cast<uint32_t>((kr * ldb + col) * 2) : kOff;
    }
    const uint32_t ring_lds = lds_addr(ring);
    const uint32_t wave_s = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(wave));
    const uint32_t w0 = __builtin_amdgcn_readfirstlane(ring_lds + wave_s * (kDma * 1024u));
    // a row-contiguous load of the slab at k0 addresses the buffer from k-row k0 on: the
    // descriptor's base moves by k0 rows and its size shrinks to match, so a k-row past K (the
    // lane's fixed offset at or past the remaining size) reads zeros, with no per-lane work
    auto rc_rsrc = [&](const int32x4 &r, int64_t k0, int64_t ld) {
        const uint64_t shift = static_cast<uint64_t>(k0 * ld * 2);
        const uint64_t base = (static_cast<uint64_t>(static_cast<uint32_t>(r.x)) |
                               (static_cast<uint64_t>(static_cast<uint32_t>(r.y) & 0xffffu) << 32)) + shift;
        int32x4 o;
        o.x = static_cast<int>(static_cast<uint32_t>(base));
        o.y = static_cast<int>(static_cast<uint32_t>(base >> 32) & 0xffffu);
        o.z = static_cast<int>(static_cast<uint32_t>(r.z) - static_cast<uint32_t>(shift));
        o.w = r.w;
        return o;
    };
    auto issue_a = [&](int sl, int i) {
        const int q = sl >= spq ? 1 : 0;
        const int64_t k0 = static_cast<int64_t>(sl - q * spq) * kSlabK;
        uint32_t dst = w0 + static_cast<uint32_t>((2 * sl) % kUnits) * kUnit;
        asm volatile("" : "+s"(dst));
        if constexpr (A_KC)
            dma16(q ? rsrc_a1 : rsrc_a0, dst + static_cast<uint32_t>(i) * 1024u, offa[i],
                  static_cast<uint32_t>(k0 * 2));
        else
            dma16(rc_rsrc(q ? rsrc_a1 : rsrc_a0, k0, lda), dst + static_cast<uint32_t>(i) * 1024u, offa[i], 0u);
    };
    auto issue_b = [&](int sl, int i) {
        const int q = sl >= spq ? 1 : 0;
        const int64_t k0 = static_cast<int64_t>(sl - q * spq) * kSlabK;
        uint32_t dst = w0 + static_cast<uint32_t>((2 * sl + 1) % kUnits) * kUnit;
        asm volatile("" : "+s"(dst));
        dma16(rc_rsrc(q ? rsrc_b1 : rsrc_b0, k0, ldb), dst + static_cast<uint32_t>(i) * 1024u, offb[i], 0u);
    };
    auto unit_a = [&](int sl) { return ring + ((2 * sl) % kUnits) * kUnit; };
    auto unit_b = [&](int sl) { return ring + ((2 * sl + 1) % kUnits) * kUnit; };

    struct Frag {
        bf16x8 s[kSubS], r[kSubR];
    };
    uint32_t soff[kSubS], roff[A_KC ? 1 : kSubR];
#pragma unroll
    for (int x = 0; x < kSubS; ++x) soff[x] = rc_lane_off(ws * kWS + 32 * x, lane);
    if constexpr (!A_KC) {
#pragma unroll
        for (int y = 0; y < kSubR; ++y) roff[y] = rc_lane_off(wr * 128 + 32 * y, lane);
    }
    // fragment part p of k-step ks: column subtile p (p < kSubS) or row subtile p - kSubS
    auto load_part = [&](const uint8_t *ua, const uint8_t *ub, int ks, Frag &f, int p) {
        if (p < kSubS) {
            f.s[p] = rc_frag(ub, ks, soff[p]);
        } else {
            const int y = p - kSubS;
            if constexpr (A_KC)
                f.r[y] = kc_frag(ua, ks, wr * 128 + 32 * y + (lane & 31), lane);
            else
                f.r[y] = rc_frag(ua, ks, roff[y]);
        }
    };
    // parts in the order the next k-step's MFMAs first use them: s0, r0 .. r3, s1 ..
    auto part_of = [](int q) { return q == 0 ? 0 : (q <= kSubR ? kSubS + q - 1 : q - kSubR); };

    floatx16 acc[kSubS][kSubR];
#pragma unroll
    for (int x = 0; x < kSubS; ++x)
#pragma unroll
        for (int y = 0; y < kSubR; ++y)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[x][y][e] = 0.f;

#pragma unroll
    for (int i = 0; i < kDma; ++i) issue_a(0, i);
#pragma unroll
    for (int i = 0; i < kDma; ++i) issue_b(0, i);
    if (slabs > 1) {
#pragma unroll
        for (int i = 0; i < kDma; ++i) issue_a(1, i);
#pragma unroll
        for (int i = 0; i < kDma; ++i) issue_b(1, i);
        wait_vmcnt<2 * kDma>();
    } else {
        wait_vmcnt<0>();
    }
    __syncthreads();
    Frag f0, f1;
#pragma unroll
    for (int q = 0; q < kParts; ++q) load_part(unit_a(0), unit_b(0), 0, f0, part_of(q));

    auto mfma = [&](const Frag &f, int i) {
        acc[i / kSubR][i % kSubR] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            f.s[i / kSubR], f.r[i % kSubR], acc[i / kSubR][i % kSubR], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    };
    // Slab s, four k-steps: each k-step's MFMAs run while the next one's fragments are read.
    // k-steps 0 and 1 issue A_{s+2} (into B_{s-1}'s unit, free since the previous barrier).
    // k-step 3 waits for slab s+1 after its first kPre MFMAs, passes the barrier (every wave has
    // read all of slab s), then issues B_{s+2} (into A_s's unit) and reads slab s+1's k-step 0.
    auto slab = [&](int sl, auto wait, auto dma) {
        const uint8_t *ua = unit_a(sl), *ub = unit_b(sl);
#pragma unroll
        for (int ks = 0; ks < 3; ++ks) {
            Frag &cur = ks % 2 == 0 ? f0 : f1;
            Frag &nxt = ks % 2 == 0 ? f1 : f0;
#pragma unroll
            for (int i = 0; i < kMfma; ++i) {
                mfma(cur, i);
                const int dq = ks * kMfma + i;  // A loads: one per MFMA slot of k-steps 0 and 1
                if (decltype(dma)::value && ks < 2 && dq % (2 * kMfma / kDma) == 0 &&
                    dq / (2 * kMfma / kDma) < kDma) {
                    issue_a(sl + 2, dq / (2 * kMfma / kDma));
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (i < kParts) {
                    load_part(ua, ub, ks + 1, nxt, part_of(i));
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
        // k-step 3 (fragments in f1)
#pragma unroll
        for (int i = 0; i < kPre; ++i) mfma(f1, i);
        if constexpr (decltype(wait)::value == 1) wait_vmcnt<kDma>();  // A_{s+2} may still fly
        if constexpr (decltype(wait)::value == 2) wait_vmcnt<0>();
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t *na = unit_a(sl + 1), *nb = unit_b(sl + 1);
        constexpr int kSpreadB = (kMfma - kPre) >= kDma ? (kMfma - kPre) / kDma : 1;
#pragma unroll
        for (int i = kPre; i < kMfma; ++i) {
            mfma(f1, i);
            const int q = i - kPre;
            if (decltype(dma)::value) {
                // B loads: one per MFMA slot, the ones left over after the last MFMA
#pragma unroll
                for (int d = 0; d < kDma; ++d)
                    if ((d / kSpreadB == q && d / kSpreadB < kMfma - kPre - 1) ||
                        (q == kMfma - kPre - 1 && d / kSpreadB >= kMfma - kPre - 1)) {
                        issue_b(sl + 2, d);
                        __builtin_amdgcn_sched_barrier(0);
                    }
            }
            if (q < kParts) {  // past the last slab these read a stale unit; unused
                load_part(na, nb, 0, f0, part_of(q));
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    using WaitA = std::integral_constant<int, 1>;
    using WaitAll = std::integral_constant<int, 2>;
    using NoWait = std::integral_constant<int, 0>;
    for (int sl = 0; sl + 2 < slabs; ++sl) slab(sl, WaitA{}, std::true_type{});
    if (slabs >= 2) slab(slabs - 2, WaitAll{}, std::false_type{});
    slab(slabs - 1, NoWait{}, std::false_type{});
    __syncthreads();  // every wave is done with the ring

    // ---- epilogue: acc[x][y][4 g + e] is C[row 32 y + (lane & 31)][column 32 x + 8 g + 4 (lane >> 5) + e]
    // of the wave's 128 x kWS tile; staged as bf16 rows, then stored as 16-byte row chunks
    uint8_t *stage = ring + wave * (128 * kPitch);
    {
        const int tr = lane & 31, half = lane >> 5;
#pragma unroll
        for (int x = 0; x < kSubS; ++x)
#pragma unroll
            for (int y = 0; y < kSubR; ++y)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    uint32_t w[2];
                    uint16_t *tv = reinterpret_cast<uint16_t *>(w);
#pragma unroll
                    for (int e = 0; e < 4; ++e) tv[e] = float_to_bf16_bits_rne(acc_read(acc[x][y], 4 * g + e));
                    *reinterpret_cast<uint2 *>(stage + (32 * y + tr) * kPitch + (32 * x + 8 * g + 4 * half) * 2) =
                        make_uint2(w[0], w[1]);
                }
    }
    __syncthreads();
    constexpr int kChunksPerRow = kWS / 8;
    constexpr int kIters = 128 * kChunksPerRow / 64;
    uint16_t *c = a.c[prob];
#pragma unroll 4
    for (int it = 0; it < kIters; ++it) {
        const int ch = it * 64 + lane;
        const int row = ch / kChunksPerRow, cc = ch - (ch / kChunksPerRow) * kChunksPerRow;
        const int64_t rg = r0 + wr * 128 + row;
        const int64_t sg = s0 + ws * kWS + cc * 8;
        const u32x4_v v = *reinterpret_cast<const u32x4_v *>(stage + row * kPitch + cc * 16);
        if (rg < a.R && sg < a.S) *as_global(reinterpret_cast<u32x4_v *>(c + rg * a.ldc + sg)) = v;
    }
}

__global__ __launch_bounds__(kThreads) void zero_u16_kernel(uint16_t *p, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t k = i; k < n; k += stride) p[k] = 0;
}

template <bool A_KC, int TS>
int launch(LgArgs &args, hipStream_t s) {
    args.n_rt = static_cast<int>(ceil_div(args.R, kTileR));
    args.n_st = static_cast<int>(ceil_div(args.S, TS));
    args.total = args.problems * args.n_rt * args.n_st;
    args.per_xcd = static_cast<int>(ceil_div(args.total, kXcds));
    hipLaunchKernelGGL((linear_grad_kernel<A_KC, TS>), dim3(static_cast<unsigned>(args.per_xcd * kXcds)),
                       dim3(kThreads), 0, s, args);
    return check_launch("me_linear_grads");
}

bool aligned16(const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace
}  // namespace me

using namespace me;

extern "C" int me_linear_grads(const void *grad_key, const void *grad_value, int64_t n, int64_t model_dim,
                               const void *mem, int64_t mem_dim, const void *w_key, const void *w_value,
                               void *grad_mem, void *grad_w_key, void *grad_w_value, void *stream) {
    ME_CHECK_ARG(n >= 0, "n must be non-negative");
    ME_CHECK_ARG(model_dim >= 8 && model_dim % 8 == 0, "model_dim must be a positive multiple of 8");
    ME_CHECK_ARG(mem_dim >= 8 && mem_dim % 8 == 0, "mem_dim must be a positive multiple of 8");
    const int64_t lim = int64_t{1} << 31;
    ME_CHECK_ARG(n * model_dim * 2 < lim && n * mem_dim * 2 < lim && model_dim * mem_dim * 2 < lim,
                 "operands must be under 2 GiB");
    ME_CHECK_ARG(grad_mem == nullptr || model_dim % 64 == 0,
                 "grad_mem needs model_dim to be a multiple of 64");
    const bool any_w = grad_w_key != nullptr || grad_w_value != nullptr;
    ME_CHECK_ARG(n == 0 || ((grad_mem == nullptr && !any_w) || (grad_key && grad_value)),
                 "grad_key and grad_value are needed");
    ME_CHECK_ARG(grad_mem == nullptr || n == 0 || (w_key && w_value), "w_key and w_value are needed");
    ME_CHECK_ARG(!any_w || n == 0 || mem, "mem is needed");
    for (const void *p : {grad_key, grad_value, mem, w_key, w_value, static_cast<const void *>(grad_mem),
                          static_cast<const void *>(grad_w_key), static_cast<const void *>(grad_w_value)})
        ME_CHECK_ARG(p == nullptr || aligned16(p), "every tensor must be 16-byte aligned");
    hipStream_t s = as_stream(stream);
    const uint32_t g_bytes = static_cast<uint32_t>(n * model_dim * 2);
    if (grad_mem != nullptr && n > 0) {
        LgArgs args{};
        args.a[0] = {grad_key, g_bytes, model_dim};
        args.a[1] = {grad_value, g_bytes, model_dim};
        const uint32_t w_bytes = static_cast<uint32_t>(model_dim * mem_dim * 2);
        args.b[0] = {w_key, w_bytes, mem_dim};
        args.b[1] = {w_value, w_bytes, mem_dim};
        args.c[0] = args.c[1] = static_cast<uint16_t *>(grad_mem);
        args.ldc = mem_dim;
        args.R = n;
        args.S = mem_dim;
        args.K = model_dim;
        args.ksegs = 2;
        args.problems = 1;
        const int rc = launch<true, 192>(args, s);
        if (rc != ME_OK) return rc;
    }
    if (!any_w) return ME_OK;
    if (n == 0) {  // an empty reduction: zero weight gradients
        for (void *p : {grad_w_key, grad_w_value}) {
            if (p == nullptr) continue;
            const int64_t cnt = model_dim * mem_dim;
            const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(ceil_div(cnt, kThreads), 4096));
            hipLaunchKernelGGL(zero_u16_kernel, dim3(blocks), dim3(kThreads), 0, s, static_cast<uint16_t *>(p), cnt);
            const int rc = check_launch("me_linear_grads");
            if (rc != ME_OK) return rc;
        }
        return ME_OK;
    }
    LgArgs args{};
    const uint32_t m_bytes = static_cast<uint32_t>(n * mem_dim * 2);
    int p = 0;
    if (grad_w_key != nullptr) {
        args.a[p] = {grad_key, g_bytes, model_dim};
        args.b[p] = {mem, m_bytes, mem_dim};
        args.c[p++] = static_cast<uint16_t *>(grad_w_key);
    }
    if (grad_w_value != nullptr) {
        args.a[p] = {grad_value, g_bytes, model_dim};
        args.b[p] = {mem, m_bytes, mem_dim};
        args.c[p++] = static_cast<uint16_t *>(grad_w_value);
    }
    if (p == 1) {
        args.a[1] = args.a[0];
        args.b[1] = args.b[0];
        args.c[1] = args.c[0];
    }
    args.ldc = mem_dim;
    args.R = model_dim;
    args.S = mem_dim;
    args.K = n;
    args.ksegs = 1;
    args.problems = p;
    return launch<false, 256>(args, s);
}
