/*
 * micro_engram.h -- C-ABI of the MI355X (gfx950) Engram lookup path.
 *
 * One shared library, libmicro_engram_amd.so, exports these entry points. They replace the
 * torch-op bodies of micro-engram's hot path (reference files cited per function). Rules that
 * hold for every entry point:
 *
 *   - Every tensor argument is a DEVICE pointer to memory the caller allocated, laid out
 *     row-major and contiguous unless a stride argument says otherwise.
 *   - Work is enqueued on `stream` (a hipStream_t passed as void*; NULL = the null stream).
 *     Nothing synchronises the host, nothing allocates device memory: a kernel that needs
 *     scratch memory takes a caller-provided workspace whose size a *_workspace_size call
 *     reports.
 *   - The return value is ME_OK (0) or a negative ME_ERR_* code; me_last_error() returns
 *     the message of the calling thread's last failure.
 *   - The library is stateless and reentrant. Calls on different streams may overlap.
 *
 * Terms. A "table set" is the n_tables embedding tables of one engram, ordered order-major,
 * head-minor (table k has n-gram order table_orders[k] and table_rows[k] rows of `dim`
 * elements). `mults` is the engram's int64 [n_tables, max_order] hash-multiplier buffer.
 */
#ifndef MICRO_ENGRAM_H
#define MICRO_ENGRAM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes -------------------------------------------------------------------- */
#define ME_OK 0
#define ME_ERR_INVALID -1     /* bad argument (shape, size, null pointer, dtype) */
#define ME_ERR_UNSUPPORTED -2 /* valid request this library has no kernel for */
#define ME_ERR_HIP -3         /* the HIP runtime reported an error (launch, stream) */
#define ME_ERR_WORKSPACE -4   /* workspace missing or smaller than *_workspace_size */

/* ---- element types ------------------------------------------------------------------- */
#define ME_I32 1
#define ME_I64 2
#define ME_F32 3
#define ME_BF16 4
#define ME_U8 5 /* bool masks */

/* ---- gate modes (module.py:49-50) ---------------------------------------------------- */
#define ME_GATE_SCALAR 0      /* sigmoid(rms(h) . rms(K) / sqrt(d)) */
#define ME_GATE_SCALAR_SQRT 1 /* learnable RMSNorm scales + signed square root of the score */

/* ---- limits -------------------------------------------------------------------------- */
#define ME_MAX_TABLES 64
#define ME_MAX_ORDER 8

/* Message of the calling thread's last failed call ("" if none). */
const char *me_last_error(void);

/* Library ABI version (bumped on any signature change). */
int me_version(void);

/*
 * me_hash_ngrams -- n-gram row ids straight from token ids.
 * Replaces MicroEngram.hash_ids (micro_engram/module.py:183-205).
 *
 *   input_ids      [batch, seq_len] of ids_dtype (ME_I32 / ME_I64)
 *   position_ids   nullable; pos_dtype ME_I32/ME_I64; element (b, t) at
 *                  position_ids[b * pos_batch_stride + t] (stride 0 broadcasts one row,
 *                  like position_ids.expand_as(ids) in the reference)
 *   canon          int64 [vocab], or NULL for the identity map (canon[i] == i, the buffer the
 *                  reference builds when no canon map is given, module.py:101-107); ids are
 *                  clamped to [0, vocab) before the lookup
 *   mults          int64 [n_tables, max_order]
 *   table_orders   HOST int32 [n_tables]; table_rows HOST int64 [n_tables]
 *   idx_out        int64 [n_tables, batch * seq_len]: idx_out[k][b*seq_len+t] is the row of
 *                  table k for the n-gram ending at (b, t)
 *
 * Token (b, t-i) enters the n-gram when t-i >= 0 and (no positions or position >= i);
 * otherwise the raw pad_id does. Hash: (sum_i token_i * mults[k][i]) mod (2^31-1) mod rows,
 * in wrapping int64 arithmetic with floor modulo, bit-exact with the reference.
 */
int me_hash_ngrams(const void *input_ids, int ids_dtype, int64_t batch, int64_t seq_len,
                   const void *position_ids, int pos_dtype, int64_t pos_batch_stride,
                   const int64_t *canon, int64_t vocab, const int64_t *mults, int32_t max_order,
                   int32_t n_tables, const int32_t *table_orders, const int64_t *table_rows,
                   int64_t pad_id, int64_t *idx_out, void *stream);

/*
 * me_hash_prev -- the same row ids from a [n, width] matrix of each token and its
 * predecessors (column i = token at t-i, negative = missing, hashed as the raw pad_id).
 * Replaces MicroEngram.hash_prev (micro_engram/module.py:207-226), the serving path fed by
 * micro_engram_vllm/ids.py:10-59. Requires width >= max_order; rows are row_stride apart.
 */
int me_hash_prev(const void *ids, int ids_dtype, int64_t n, int64_t width, int64_t row_stride,
                 const int64_t *canon, int64_t vocab, const int64_t *mults, int32_t max_order,
                 int32_t n_tables, const int32_t *table_orders, const int64_t *table_rows,
                 int64_t pad_id, int64_t *idx_out, void *stream);

/*
 * me_gather -- concatenated table rows for given row ids.
 * Replaces MicroEngram.lookup + torch.cat (micro_engram/module.py:146-154, 233) and the
 * TP=1 serving lookup micro_engram_vllm/tp.py:20-39: a row id outside [0, table_rows[k])
 * yields a zero row, as the masked lookup there does.
 *
 *   idx     int64; row ids of table k for token i at idx[k * idx_table_stride + i]
 *   tables  HOST array of n_tables device pointers, table k is [table_rows[k], dim]
 *   mem     [n, n_tables * dim] of dtype (ME_BF16 / ME_F32): mem[i][k*dim + c] = tables[k][row][c]
 */
int me_gather(const int64_t *idx, int64_t idx_table_stride, int64_t n, int32_t n_tables,
              const void *const *tables, const int64_t *table_rows, int32_t dim, int dtype,
              void *mem, void *stream);

/*
 * me_hash_gather -- me_hash_ngrams fused with me_gather: one kernel reads the token ids,
 * hashes every (token, table) pair and writes the token's concatenated memory vector.
 * Replaces MicroEngram.forward's hash_ids + lookup + cat (module.py:263-265, 183-205,
 * 146-154, 233). idx_out is nullable (row ids are written only when it is given).
 */
int me_hash_gather(const void *input_ids, int ids_dtype, int64_t batch, int64_t seq_len,
                   const void *position_ids, int pos_dtype, int64_t pos_batch_stride,
                   const int64_t *canon, int64_t vocab, const int64_t *mults, int32_t max_order,
                   int32_t n_tables, const int32_t *table_orders, const int64_t *table_rows,
                   int64_t pad_id, const void *const *tables, int32_t dim, int dtype, void *mem,
                   int64_t *idx_out, void *stream);

/*
 * me_hash_prev_gather -- me_hash_prev fused with me_gather (serving decode / chunked
 * prefill: module.py:207-226 then 146-154). idx_out is nullable.
 */
int me_hash_prev_gather(const void *ids, int ids_dtype, int64_t n, int64_t width,
                        int64_t row_stride, const int64_t *canon, int64_t vocab,
                        const int64_t *mults, int32_t max_order, int32_t n_tables,
                        const int32_t *table_orders, const int64_t *table_rows, int64_t pad_id,
                        const void *const *tables, int32_t dim, int dtype, void *mem,
                        int64_t *idx_out, void *stream);

/*
 * me_gate_workspace_size -- bytes of workspace me_gate_residual needs for n tokens of
 * model_dim (per-token partial sums of the gate, one triple per column tile of 224, the
 * narrower of the two tilings, and the per-token gates).
 */
int me_gate_workspace_size(int64_t n, int64_t model_dim, size_t *bytes);

/*
 * me_gate_residual -- key/value projection + scalar / scalar_sqrt gate + residual add.
 * Replaces MicroEngram.inject after the lookup (micro_engram/module.py:239-261):
 *
 *   K = W_K mem, V = W_V mem        (engram dtype, fp32 accumulation, rounded to dtype)
 *   h = rms_norm(hidden) [* (1 + q_scale_delta)], k = rms_norm(K) [* (1 + k_scale_delta)]
 *   s = sum(h k) / sqrt(model_dim); ME_GATE_SCALAR_SQRT: s = sign(s) sqrt(max(|s|, 1e-6))
 *   out = hidden + round_hidden(sigmoid(s) * V * keep)
 *
 *   hidden, out   [n, model_dim] of hidden_dtype (out may equal hidden: in-place is allowed)
 *   mem           [n, mem_dim] of dtype; w_key, w_value [model_dim, mem_dim] of dtype
 *                 (nn.Linear weights); mem_dim * element size must be a multiple of 16 bytes,
 *                 model_dim a multiple of 8, every tensor 16-byte aligned
 *   q/k_scale_delta  [model_dim] of scale_dtype, the stored scale - 1 (module.py:156-164);
 *                 ignored for ME_GATE_SCALAR
 *   keep          nullable [n] uint8 (bool): 0 leaves the token's hidden state unchanged
 *   alpha_out     nullable [n] fp32: the gate value of each token (before keep)
 *   row_stats     nullable [n, 4] fp32: per token sum hidden^2, sum K^2, sum hidden * (1 +
 *                 q_scale_delta) * (1 + k_scale_delta) * K (scales 1 for ME_GATE_SCALAR) and the
 *                 gate: what me_gate_backward needs of the forward
 *   workspace     at least me_gate_workspace_size(n, model_dim) bytes
 */
int me_gate_residual(const void *hidden, int hidden_dtype, int64_t n, int64_t model_dim,
                     const void *mem, int64_t mem_dim, const void *w_key, const void *w_value,
                     int dtype, const void *q_scale_delta, const void *k_scale_delta,
                     int scale_dtype, int gate_mode, const uint8_t *keep, void *out,
                     float *alpha_out, float *row_stats, void *workspace, size_t workspace_size,
                     void *stream);

/*
 * me_gate_residual_noalloc -- me_gate_residual without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops that forbid
 * allocation). It has no counterpart in the reference. Same arguments and results as
 * me_gate_residual, the same kernels; the workspace is a static 4 MiB device array of the
 * library, one per GPU, held until the process ends. It allocates nothing: n tokens of model_dim
 * need (3 ceil(model_dim / 224) + 1) * 4 * n bytes of it (at most 14,364 tokens at model dim
 * 5376); larger calls return ME_ERR_INVALID and launch nothing. The current device must be the
 * one the tensors and the stream belong to. Calls that overlap on one GPU share the array and
 * race: serialise them (one stream, or events).
 */
int me_gate_residual_noalloc(const void *hidden, int hidden_dtype, int64_t n, int64_t model_dim,
                             const void *mem, int64_t mem_dim, const void *w_key,
                             const void *w_value, int dtype, const void *q_scale_delta,
                             const void *k_scale_delta, int scale_dtype, int gate_mode,
                             const uint8_t *keep, void *out, float *alpha_out, float *row_stats,
                             void *stream);

/*
 * me_kv_proj -- the key and value projections of the memory vectors for few tokens: the two
 * nn.Linear calls of MicroEngram.inject (micro_engram/module.py:245, 254), in the engram dtype
 * with fp32 accumulation, written side by side for me_gate_rows:
 *
 *   kv[i][j] = round(sum_m mem[i][m] w_key[j][m]),  kv[i][d + j] = round(sum_m mem[i][m] w_value[j][m])
 *
 *   mem       [n, mem_dim] of dtype (ME_BF16 / ME_F32); w_key, w_value [model_dim, mem_dim]
 *   kv        [n, 2 model_dim] of dtype
 * model_dim a multiple of 8, mem_dim * element size a multiple of 16 bytes, every tensor
 * 16-byte aligned, mem and each weight under 2 GiB. Meant for batches up to a few thousand
 * tokens (a serving decode step); larger ones belong to me_gate_residual.
 */
int me_kv_proj(const void *mem, int64_t n, int64_t mem_dim, const void *w_key, const void *w_value,
               int64_t model_dim, int dtype, void *kv, void *stream);

/*
 * me_gate_rows -- the gate and residual add of me_gate_residual from key and value projections
 * computed elsewhere (few-token batches: me_kv_proj's output, where me_gate_residual's
 * 256-token tiles would leave most of the part idle). Replaces the rest of
 * MicroEngram.inject after the two nn.Linear calls (micro_engram/module.py:240-261), with the
 * same arithmetic as me_gate_residual:
 *
 *   h = rms_norm(hidden) [* (1 + q_scale_delta)], k = rms_norm(K) [* (1 + k_scale_delta)]
 *   s = sum(h k) / sqrt(model_dim); ME_GATE_SCALAR_SQRT: s = sign(s) sqrt(max(|s|, 1e-6))
 *   out = hidden + round_hidden(sigmoid(s) * V * keep)
 *
 *   hidden, out   [n, model_dim] of hidden_dtype (out may equal hidden)
 *   k_proj, v_proj  rows of K and V (dtype), kv_stride elements apart (e.g. the two halves of
 *                 one [n, 2 model_dim] GEMM output); any model_dim >= 1 and kv_stride >=
 *                 model_dim (16-byte accesses when both are multiples of 8 and every tensor is
 *                 16-byte aligned, element accesses otherwise: an engram of any model dim)
 *   q/k_scale_delta, keep, alpha_out, row_stats   as for me_gate_residual
 */
int me_gate_rows(const void *hidden, int hidden_dtype, int64_t n, int64_t model_dim,
                 const void *k_proj, const void *v_proj, int64_t kv_stride, int dtype,
                 const void *q_scale_delta, const void *k_scale_delta, int scale_dtype,
                 int gate_mode, const uint8_t *keep, void *out, float *alpha_out,
                 float *row_stats, void *stream);

/*
 * me_gate_rows_backward_workspace_size -- bytes of workspace me_gate_rows_backward needs.
 */
int me_gate_rows_backward_workspace_size(int64_t n, int64_t model_dim, size_t *bytes);

/*
 * me_gate_rows_backward -- gradients of me_gate_rows from the same K and V rows: what autograd
 * computes through MicroEngram.inject after its two nn.Linear calls (micro_engram/module.py:
 * 239-261), the arithmetic of me_gate_backward (which recomputes K and V on MFMA tiles, for the
 * shapes those take) for any model dim:
 *
 *   dV = round(alpha keep g);  d alpha = keep sum g V;  ds = d alpha alpha (1 - alpha)
 *   ds0 = ds / (2 sqrt|s0|) where |s0| >= 1e-6, else 0 (ME_GATE_SCALAR_SQRT); ds (ME_GATE_SCALAR)
 *   a = ds0 r_h r_k / sqrt(d); d hidden = g + round(a w K - a r_h^2 sck / d x)
 *   dK = round(a w x - a r_k^2 sck / d K);  d q_scale_delta_j = ks_j P_j, d k_scale_delta_j = qs_j P_j
 *   with w = qs ks, P_j = sum over tokens of a x_j K_j
 *
 *   hidden, grad_out, grad_hidden   [n, model_dim] of hidden_dtype
 *   k_proj, v_proj  the forward's K and V rows (dtype), kv_stride elements apart
 *   row_stats     [n, 4] fp32 of the forward (me_gate_rows or me_gate_residual on the same K, V)
 *   grad_key, grad_value   [n, model_dim] of dtype: the gradients of the Linear outputs K and V
 *   grad_q_scale, grad_k_scale   [model_dim] fp32 (ME_GATE_SCALAR_SQRT only)
 *   workspace     at least me_gate_rows_backward_workspace_size(n, model_dim) bytes
 */
int me_gate_rows_backward(const void *hidden, int hidden_dtype, int64_t n, int64_t model_dim,
                          const void *k_proj, const void *v_proj, int64_t kv_stride, int dtype,
                          const void *q_scale_delta, const void *k_scale_delta, int scale_dtype,
                          int gate_mode, const uint8_t *keep, const void *grad_out,
                          const float *row_stats, void *grad_hidden, void *grad_key,
                          void *grad_value, float *grad_q_scale, float *grad_k_scale,
                          void *workspace, size_t workspace_size, void *stream);

/*
 * me_gate_backward_workspace_size -- bytes of workspace me_gate_backward needs.
 */
int me_gate_backward_workspace_size(int64_t n, int64_t model_dim, size_t *bytes);

/*
 * me_gate_backward -- gradients of me_gate_residual: what autograd computes through
 * MicroEngram.inject (micro_engram/module.py:239-261) for the scalar gates, given the gradient
 * of its output. The projections K and V are recomputed (same MFMA tiles as the forward), so
 * the forward keeps only row_stats.
 *
 *   same shapes, dtypes and rules as me_gate_residual for hidden .. keep
 *   grad_out      [n, model_dim] of hidden_dtype: gradient of out
 *   row_stats     [n, 4] fp32 from the forward (me_gate_residual's row_stats)
 *   grad_hidden   [n, model_dim] of hidden_dtype: grad_out + the gradient through the gate's
 *                 rms norm of hidden, rounded to hidden_dtype first (hidden.float()'s backward)
 *   grad_key      [n, model_dim] of dtype: gradient of K = W_K mem (the key Linear's output)
 *   grad_value    [n, model_dim] of dtype: gradient of V = W_V mem; the weight and mem
 *                 gradients are then plain GEMMs: dW_K = grad_key^T mem, dW_V = grad_value^T mem,
 *                 dmem = grad_key W_K + grad_value W_V
 *   grad_q/k_scale  [model_dim] fp32: gradients of q_scale_delta / k_scale_delta (needed for
 *                 ME_GATE_SCALAR_SQRT, ignored otherwise)
 *   workspace     at least me_gate_backward_workspace_size(n, model_dim) bytes
 */
int me_gate_backward(const void *hidden, int hidden_dtype, int64_t n, int64_t model_dim,
                     const void *mem, int64_t mem_dim, const void *w_key, const void *w_value,
                     int dtype, const void *q_scale_delta, const void *k_scale_delta,
                     int scale_dtype, int gate_mode, const uint8_t *keep, const void *grad_out,
                     const float *row_stats, void *grad_hidden, void *grad_key, void *grad_value,
                     float *grad_q_scale, float *grad_k_scale, void *workspace,
                     size_t workspace_size, void *stream);

/*
 * me_dedup_workspace_size -- bytes of workspace me_dedup needs for n keys.
 */
int me_dedup_workspace_size(int64_t n, size_t *bytes);

/*
 * me_linear_grads -- gradients of the engram's key / value Linear layers from the gradients of
 * their outputs (what autograd computes for the two nn.Linear calls of the reference's forward,
 * micro_engram/module.py:245, 254; here after me_gate_backward):
 *
 *   grad_mem     [n, mem_dim]   = grad_key . w_key + grad_value . w_value
 *   grad_w_key   [model_dim, mem_dim] = grad_key^T . mem;  grad_w_value = grad_value^T . mem
 *
 *   grad_key, grad_value   [n, model_dim] bf16 (me_gate_backward's outputs)
 *   mem           [n, mem_dim] bf16, w_key / w_value [model_dim, mem_dim] bf16
 *   outputs bf16, any of them NULL to skip it; fp32 accumulation over the whole reduction (both
 *   products of grad_mem in one sum), one round to nearest even per element. n == 0 leaves
 *   zero weight gradients. model_dim and mem_dim multiples of 8 (of 64 for grad_mem), every
 *   operand under 2 GiB and 16-byte aligned.
 */
int me_linear_grads(const void *grad_key, const void *grad_value, int64_t n, int64_t model_dim,
                    const void *mem, int64_t mem_dim, const void *w_key, const void *w_value,
                    void *grad_mem, void *grad_w_key, void *grad_w_value, void *stream);

/*
 * me_dedup -- touched-row dedup with coalesced gradients.
 * Replaces torch.unique(flat, return_inverse=True) and zeros(n_uniq, D).index_add_(0, inv, g)
 * (micro_engram/rows.py:81, 117-118; add_sparse_grad rows.py:137-147).
 *
 *   keys       int64 [n], every key in [0, key_bound) (table offset + row)
 *   grads      nullable [n, dim] of grad_dtype (ME_F32 / ME_BF16): the gradient row of each key
 *   uniq       int64 [n]: the count unique keys, ascending, in uniq[0 .. count)
 *   inv        int64 [n]: uniq[inv[i]] == keys[i]
 *   gsum       fp32 [n, dim] (needed when grads is given): row u = fp32 sum of the grads of the
 *              keys equal to uniq[u], added in increasing i from +0.0 (bit-exact with CPU
 *              index_add_)
 *   count      int64 [1], device: the number of unique keys
 */
int me_dedup(const int64_t *keys, int64_t n, int64_t key_bound, const void *grads, int grad_dtype,
             int32_t dim, int64_t *uniq, int64_t *inv, float *gsum, int64_t *count,
             void *workspace, size_t workspace_size, void *stream);

/*
 * me_dedup_table_bounds -- where each table's rows lie in the unique keys of an me_dedup_keys
 * call over concatenated-table keys (table offset + row): the bounds rows.py:123-129 splits the
 * unique rows and sums by, and each unique key's row in its own table (the searchsorted of the
 * keys against the table offsets), in one launch:
 *
 *   local_rows[i] = uniq[i] - table_offsets[t]     t = the table of uniq[i], i < *count
 *   info[0] = *count;  info[1 + t] = number of unique keys below table_offsets[t], t <= n_tables
 *
 *   uniq          [n] int64 ascending (valid up to *count); count  device int64 scalar
 *   table_offsets n_tables + 1 host int64 values, ascending, from 0 (the last: the key bound)
 *   local_rows    [n] int64 (entries past the count are left as they are)
 *   info          [n_tables + 2] int64 device
 */
int me_dedup_table_bounds(const int64_t *uniq, int64_t n, const int64_t *count,
                          const int64_t *table_offsets, int32_t n_tables, int64_t *local_rows,
                          int64_t *info, void *stream);

/*
 * me_dedup_tables -- the key half of a row lookup's dedup from its per-table row ids, and the
 * tables' bounds in it: what me_dedup_keys + me_dedup_table_bounds give for the token-major keys
 * offset_k + idx[k][t] (lookup position t * n_tables + k), in two launches for up to 8,192
 * tokens (micro_engram/rows.py:81 torch.unique(return_inverse=True) over the lookups' keys, and
 * the per-table slices of rows.py:123-129). Every table holds n lookups, so table k's part of the
 * sorted order is [k * n, (k + 1) * n): each workgroup takes one range of one table's rows, reads
 * the table's ids, and sorts its lookups where they land; a second launch numbers the unique keys.
 * Larger n: the keys, then the me_dedup_keys path and the bounds.
 *
 *   idx          [n_tables, idx_table_stride] int64 row ids (token t of table k at
 *                idx[k * idx_table_stride + t]); rows outside [0, table_rows[k]) are outside the
 *                contract (clamped, so nothing is written out of bounds)
 *   table_rows   n_tables host int64 row counts; offset_k = sum of the rows of tables below k
 *   uniq         [n * n_tables] int64 unique keys ascending (the first count are valid)
 *   local_rows   [n * n_tables] int64 row of each unique key in its table
 *   inv          [n * n_tables] int64 unique index of each lookup position, or null: not
 *                written (me_dedup_sums reads the plan only)
 *   info         [n_tables + 2] int64: count, the first unique index of each table, count
 *   plan         at least me_dedup_plan_size(n * n_tables) bytes, read by me_dedup_sums with
 *                count = info
 *   workspace    at least me_dedup_tables_workspace_size bytes (free again when the work ends)
 */
int me_dedup_tables_workspace_size(int64_t n, int32_t n_tables, const int64_t *table_rows,
                                   size_t *bytes);
int me_dedup_tables(const int64_t *idx, int64_t idx_table_stride, int64_t n, int32_t n_tables,
                    const int64_t *table_rows, int64_t *uniq, int64_t *local_rows, int64_t *inv,
                    int64_t *info, void *plan, size_t plan_size, void *workspace,
                    size_t workspace_size, void *stream);

/*
 * me_dedup_plan_size -- bytes of the segment plan me_dedup_keys writes for n keys.
 */
int me_dedup_plan_size(int64_t n, size_t *bytes);

/*
 * me_dedup_keys -- the key half of me_dedup: torch.unique(keys, return_inverse=True)
 * (micro_engram/rows.py:81) plus a plan of which positions form each unique key's segment, so
 * that me_dedup_sums can later add the gradient rows (rows.py:117-118) without sorting again.
 * The keys depend only on the hashed row ids: a caller may run this half as soon as the forward
 * has them, on another stream, and only the sums in the backward.
 *
 *   keys, n, key_bound, uniq, inv, count   as for me_dedup
 *   plan       device buffer of at least me_dedup_plan_size(n) bytes, read by me_dedup_sums
 *   workspace  at least me_dedup_workspace_size(n) bytes (free again when this call's work ends)
 */
int me_dedup_keys(const int64_t *keys, int64_t n, int64_t key_bound, int64_t *uniq, int64_t *inv,
                  int64_t *count, void *plan, size_t plan_size, void *workspace,
                  size_t workspace_size, void *stream);

/*
 * me_dedup_sums -- the gradient half of me_dedup: gsum row u = fp32 sum of the grads of the
 * keys equal to uniq[u], added in increasing position from +0.0 (bit-exact with CPU index_add_,
 * rows.py:117-118, 144-146), from the plan and count of an me_dedup_keys call on the same keys.
 *
 *   grads   [n, dim] of grad_dtype (ME_F32 / ME_BF16); gsum fp32 [n, dim] (rows past count unset)
 */
int me_dedup_sums(const void *plan, size_t plan_size, int64_t n, const int64_t *count,
                  const void *grads, int grad_dtype, int32_t dim, float *gsum, void *stream);

/*
 * me_sumsq -- sum of squares of n fp32 values into *out (or added to it when accumulate != 0),
 * in a fixed order. The squared gradient norm of RowTables.clip (micro_engram/rows.py:214-223).
 * workspace: at least 1 KiB.
 */
int me_sumsq(const float *x, int64_t n, float *out, int accumulate, void *workspace,
             size_t workspace_size, void *stream);

/*
 * me_clip_scale -- the in-place scaling of RowTables.clip (micro_engram/rows.py:221-231):
 * x *= coef with coef = min(max_norm * (1 / (sqrt(*sumsq) + 1e-6)), 1) in fp32 (torch evaluates
 * the reference's max_norm / (norm + 1e-6) as a reciprocal and a product; a NaN norm gives a NaN
 * coef). bf16 x is multiplied by coef rounded to bf16 (p.grad.mul_(coef.to(bf16))) and rounded.
 *
 *   x        [n] of dtype (ME_F32 / ME_BF16), 16-byte aligned, scaled in place
 *   sumsq    device fp32 scalar: the squared gradient norm (me_sumsq)
 *   max_norm > 0
 */
int me_clip_scale(void *x, int dtype, int64_t n, const float *sumsq, double max_norm, void *stream);

/*
 * me_sparse_adam -- one LazyAdamW step on the given rows of n_tables tables.
 * Replaces the row branches of LazyAdamW.step (micro_engram/optim.py:65-133): with lazy != 0,
 * rows whose gradient is all zero are skipped (optim.py:88-104); weight decay, first moment, second moment (one
 * fp32 value per row when rowwise != 0, else per value in sq_dtype), bias correction with each
 * table's own step count, and write-back of weights and moments, with stochastic rounding to bf16
 * when stochastic_rounding != 0 (optim.py:33-44).
 *
 *   HOST arrays [n_tables]: params, exp_avgs (device [rows_k, dim], param_dtype), exp_avg_sqs
 *   (device [rows_k] fp32 or [rows_k, dim] sq_dtype), rows (device int64 [n_rows_k], unique),
 *   grads (device [n_rows_k, dim] of grad_dtype, ME_F32 or ME_BF16), n_rows, steps (the step count after this step's
 *   increment), stream_ids (< 65536, distinct per table: selects the table's rounding noise)
 * The rounding noise of element (row, col) is 16 bits of Philox4x32-10 keyed by seed with counter
 * (row low, row high, step, stream_id << 16 | which << 14 | col >> 3), word (col >> 1) & 3,
 * half col & 1; which = 0 weights, 1 first moment, 2 per-value second moment.
 */
int me_sparse_adam(int32_t n_tables, void *const *params, void *const *exp_avgs,
                   void *const *exp_avg_sqs, const int64_t *const *rows, const void *const *grads,
                   int grad_dtype, const int64_t *n_rows, const int64_t *steps, const int32_t *stream_ids,
                   int32_t dim, int param_dtype, int rowwise, int sq_dtype, int lazy, double lr,
                   double beta1, double beta2, double eps, double weight_decay,
                   int stochastic_rounding, uint64_t seed, void *stream);

/*
 * me_stochastic_bf16 -- fp32 -> bf16 with stochastic rounding (micro_engram/optim.py:33-44):
 * the 16-bit noise is added to the fp32 bit pattern below the kept bits, then the low 16 bits
 * are dropped; inf and NaN convert as usual. Element i takes the me_sparse_adam noise of
 * (row i / 4096, column i % 4096, which 0) for stream_id and step. out is bf16 bits [n].
 */
int me_stochastic_bf16(const float *x, int64_t n, uint16_t *out, uint64_t seed, uint32_t step,
                       uint32_t stream_id, void *stream);

/*
 * me_fill_engram_ids -- the serving step's [tokens, max_order] matrix of each scheduled token
 * and the ones before it, -1 where there is none (the input of me_hash_prev).
 * Replaces fill_engram_ids (micro_engram_vllm/ids.py:10-59), and with media ids also
 * mask_media (ids.py:62-70) in the same launch.
 *
 *   out            int32 [out_rows, out_row_stride]; rows [0, num_tokens_padded) are written,
 *                  rows from num_tokens on are -1 (graph padding)
 *   input_ids, positions      [>= num_tokens] this step's tokens (requests back to back)
 *   idx_mapping    [>= num_reqs] request -> row of all_token_ids
 *   query_start_loc [>= num_reqs + 1] first token of each request
 *   all_token_ids  [hist_rows, hist_row_stride], hist_len valid columns: each request's tokens
 *   media_ids      nullable, n_media <= 64 ids: entries equal to one of them become -1 and
 *                  keep_out[t] (nullable, uint8 [num_tokens_padded]) is 0 where column 0 is one
 *   *_dtype        ME_I32 or ME_I64
 *
 * Token t of request r: column 0 = input_ids[t]; column k reads input_ids[t - k] when position
 * - k >= the chunk's first position, else the history row through the reference's lookback
 * index. History reads outside [0, hist_len) or a request row outside [0, hist_rows) give -1.
 */
int me_fill_engram_ids(int32_t *out, int64_t out_rows, int64_t out_row_stride, int32_t max_order,
                       const void *input_ids, int ids_dtype, const void *positions, int pos_dtype,
                       const void *idx_mapping, int map_dtype, const void *query_start_loc,
                       int qsl_dtype, const void *all_token_ids, int hist_dtype, int64_t hist_rows,
                       int64_t hist_len, int64_t hist_row_stride, int64_t num_reqs,
                       int64_t num_tokens, int64_t num_tokens_padded, const void *media_ids,
                       int media_dtype, int32_t n_media, uint8_t *keep_out, void *stream);

/*
 * me_mask_media -- media placeholder ids become -1; keep_out[t] = 0 where column 0 is one.
 * Replaces mask_media (micro_engram_vllm/ids.py:62-70).
 *
 *   ids      [n, width] of ids_dtype, rows row_stride elements apart
 *   ids_out  int32 [n, width] contiguous; keep_out uint8 [n]
 */
int me_mask_media(const void *ids, int ids_dtype, int64_t n, int64_t width, int64_t row_stride,
                  const void *media_ids, int media_dtype, int32_t n_media, int32_t *ids_out,
                  uint8_t *keep_out, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MICRO_ENGRAM_H */
