/*
 * CPU oracle -- TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the expected result the HIP path is
 * tested against.
 *
 * Plain-C restatement of the integer half of micro-engram's Engram lookup path:
 *   oracle_mt19937      the Mersenne Twister MT19937 (Matsumoto & Nishimura 1998), the engine
 *                       behind torch's CPU generator
 *   oracle_randint      torch.randint(low, high) on that engine for ranges below 2^32, the call
 *                       that makes the hash multipliers (micro_engram/module.py:94-99)
 *   oracle_hash_ids     MicroEngram.hash_ids (module.py:183-205)
 *   oracle_hash_prev    MicroEngram.hash_prev (module.py:207-226)
 *
 * The hash is written the plain way (wrapping int64 sum, C '%' with a sign fix-up for floor
 * modulo, one token at a time), deliberately unlike the GPU kernels' Mersenne folding and
 * magic-number division, so the two cannot share a mistake. The llama.cpp restatement
 * (llama_cpp/src/llama-micro-engram.cpp:150-176) computes the same sum in uint64.
 */
#include <stddef.h>
#include <stdint.h>

#define ORACLE_PRIME 2147483647LL /* 2^31 - 1 (module.py:5) */

/* ---- MT19937 ---------------------------------------------------------------------------- */
#define MT_N 624
#define MT_M 397

typedef struct {
    uint32_t s[MT_N];
    int i;
} mt_state;

static void mt_seed(mt_state *mt, uint32_t seed) {
    mt->s[0] = seed;
    for (int j = 1; j < MT_N; ++j)
        mt->s[j] = 1812433253u * (mt->s[j - 1] ^ (mt->s[j - 1] >> 30)) + (uint32_t)j;
    mt->i = MT_N;
}

static uint32_t mt_next(mt_state *mt) {
    if (mt->i >= MT_N) {
        for (int j = 0; j < MT_N; ++j) {
            uint32_t y = (mt->s[j] & 0x80000000u) | (mt->s[(j + 1) % MT_N] & 0x7fffffffu);
            uint32_t v = mt->s[(j + MT_M) % MT_N] ^ (y >> 1);
            if (y & 1u) v ^= 0x9908b0dfu;
            mt->s[j] = v;
        }
        mt->i = 0;
    }
    uint32_t y = mt->s[mt->i++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

/* The first n outputs of MT19937 seeded with `seed`. */
void oracle_mt19937(uint32_t seed, int64_t n, uint32_t *out) {
    mt_state mt;
    mt_seed(&mt, seed);
    for (int64_t i = 0; i < n; ++i) out[i] = mt_next(&mt);
}

/* torch.randint(low, high, (n,), generator=Generator().manual_seed(seed)) on the CPU: a range
 * below 2^28 takes one 32-bit engine output, a larger one a 64-bit value made of two outputs
 * (first << 32 | second); the draw is low + value % range (torch's uniform_int_from_to
 * distribution, ATen/core/DistributionsHelper.h in open-source builds). Returns -1 for
 * arguments this restatement does not cover. */
int oracle_randint(uint64_t seed, int64_t low, int64_t high, int64_t n, int64_t *out) {
    const int64_t range = high - low;
    if (range <= 0 || seed > 0xffffffffull) return -1;
    mt_state mt;
    mt_seed(&mt, (uint32_t)seed);
    for (int64_t i = 0; i < n; ++i) {
        uint64_t v;
        if (range >= (1LL << 28)) {
            const uint64_t hi = mt_next(&mt);
            v = (hi << 32) | mt_next(&mt);
        } else {
            v = mt_next(&mt);
        }
        out[i] = low + (int64_t)(v % (uint64_t)range);
    }
    return 0;
}

/* ---- hash ---------------------------------------------------------------------------------- */
static int64_t floor_mod(int64_t x, int64_t m) {
    int64_t r = x % m;
    return r < 0 ? r + m : r;
}

static int64_t canon_of(const int64_t *canon, int64_t vocab, int64_t id) {
    if (id < 0) id = 0;
    if (id > vocab - 1) id = vocab - 1;
    return canon[id];
}

static int64_t ngram_row(const int64_t *tok, const int64_t *mult, int order, int64_t rows) {
    uint64_t x = 0; /* int64 arithmetic with wrap-around, as torch's int64 tensors */
    for (int i = 0; i < order; ++i) x += (uint64_t)tok[i] * (uint64_t)mult[i];
    return floor_mod(floor_mod((int64_t)x, ORACLE_PRIME), rows);
}

/*
 * ids [batch, seq_len]; pos nullable, element (b, t) at pos[b * pos_bstride + t];
 * out [n_tables, batch * seq_len]. Returns -1 on bad arguments.
 */
int oracle_hash_ids(const int64_t *ids, int64_t batch, int64_t seq_len, const int64_t *pos,
                    int64_t pos_bstride, const int64_t *canon, int64_t vocab,
                    const int64_t *mults, int max_order, int n_tables, const int32_t *orders,
                    const int64_t *rows, int64_t pad_id, int64_t *out) {
    if (max_order < 1 || max_order > 64 || vocab < 1) return -1;
    int64_t tok[64];
    const int64_t n = batch * seq_len;
    for (int64_t b = 0; b < batch; ++b) {
        for (int64_t t = 0; t < seq_len; ++t) {
            /* tok[i] = token at t - i of the same row, or the raw pad id before the sequence
             * start or (with positions) before the document start */
            for (int i = 0; i < max_order; ++i) {
                int use = t - i >= 0;
                if (use && i > 0 && pos != NULL) use = pos[b * pos_bstride + t] >= i;
                tok[i] = use ? canon_of(canon, vocab, ids[b * seq_len + t - i]) : pad_id;
            }
            for (int k = 0; k < n_tables; ++k) {
                if (orders[k] < 1 || orders[k] > max_order || rows[k] < 1) return -1;
                out[(int64_t)k * n + b * seq_len + t] =
                    ngram_row(tok, mults + (int64_t)k * max_order, orders[k], rows[k]);
            }
        }
    }
    return 0;
}

/* ids [n, width] (column i = token at t - i, negative = missing); out [n_tables, n]. */
int oracle_hash_prev(const int64_t *ids, int64_t n, int64_t width, const int64_t *canon,
                     int64_t vocab, const int64_t *mults, int max_order, int n_tables,
                     const int32_t *orders, const int64_t *rows, int64_t pad_id, int64_t *out) {
    if (max_order < 1 || max_order > 64 || width < max_order || vocab < 1) return -1;
    int64_t tok[64];
    for (int64_t r = 0; r < n; ++r) {
        for (int i = 0; i < max_order; ++i) {
            const int64_t id = ids[r * width + i];
            tok[i] = id >= 0 ? canon_of(canon, vocab, id) : pad_id;
        }
        for (int k = 0; k < n_tables; ++k) {
            if (orders[k] < 1 || orders[k] > max_order || rows[k] < 1) return -1;
            out[(int64_t)k * n + r] = ngram_row(tok, mults + (int64_t)k * max_order, orders[k], rows[k]);
        }
    }
    return 0;
}
