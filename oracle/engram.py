"""CPU oracle of the Engram lookup path -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Function                 restates                                         pinned by (tests/)
-----------------------  -----------------------------------------------  -------------------------------
make_mults               micro_engram/module.py:94-99                     MT19937 10000th-output known
                                                                          answer; torch.randint itself
hash_ids                 micro_engram/module.py:183-205                   exact big-integer brute force;
                                                                          canon/boundary invariants of
                                                                          test_canon.py:42-56 and
                                                                          test_vllm_ids.py:68-83
hash_prev                micro_engram/module.py:207-226                   hash_prev == hash_ids
                                                                          (test_vllm_ids.py:68-83)
hash_ids_torch           micro_engram/module.py:183-205 as torch ops      == hash_ids (C), bit for bit
hash_prev_torch          micro_engram/module.py:207-226 as torch ops      == hash_prev (C), bit for bit
lookup                   module.py:146-154, micro_engram_vllm/tp.py:20-39 numpy fancy indexing identity
lookup_torch             module.py:146-154 (F.embedding + cat)            == lookup (tests of the bench's
                                                                          baseline inputs)
inject                   micro_engram/module.py:228-261                   test_oracle_inject.py: value=0
                                                                          no-op and keep mask
                                                                          (test_gate.py:24-27, 122-130);
                                                                          hidden 0 -> alpha 1/2 exactly;
                                                                          constant hidden and key ->
                                                                          closed-form s0 = sqrt(d) c c'
                                                                          r_h r_k (fp32 eps visible);
                                                                          scales multiply s0; the 1e-6
                                                                          clamp; bf16 roundings of K and
                                                                          of the add
inject_backward          autograd of micro_engram/module.py:239-261       torch.autograd of inject on the
                         (closed form, float64)                           same inputs; finite differences
                                                                          of inject in float64
dedup                    micro_engram/rows.py:81, 117-118, 137-147        brute-force Python loop on tiny
                                                                          inputs; uniq[inv] == keys
dedup_torch              micro_engram/rows.py:81, 117-118 as torch ops    the same brute force, bit for bit
philox4x32_10            Salmon et al. 2011 (Random123)                   published known-answer vectors
stochastic_bf16          micro_engram/optim.py:33-44                      exhaustive 2^16-noise count;
                                                                          fp32 pass-through, inf kept
clip_coef, clip          micro_engram/rows.py:208-233                     test_oracle_rows.py: norms of
                                                                          known gradients; coef < 1
                                                                          brings the norm to max_norm;
                                                                          coef 1 leaves them bit-equal;
                                                                          bf16 scaled by the bf16 coef
sparse_adam_step         micro_engram/optim.py:65-133 (sparse branch)     == torch.optim.AdamW when |g| is
                                                                          uniform per row
                                                                          (test_optim.py:74-80); lazy
                                                                          invariants (test_optim.py:56-65,
                                                                          84-88)
fill_engram_ids          micro_engram_vllm/ids.py:10-59                   brute-force expected() of
                                                                          test_vllm_ids.py:59-65 over its
                                                                          six step kinds (84-98)
mask_media               micro_engram_vllm/ids.py:62-70                   the multimodal cases of
                                                                          test_vllm_ids.py:135-160
"""
import ctypes
import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
PRIME = 2_147_483_647  # 2^31 - 1 (module.py:5)

_lib = None


def _c():
    """The C half of the oracle (oracle/liboracle.so, built by `make -C oracle`)."""
    global _lib
    if _lib is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run `make -C oracle`")
        lib = ctypes.CDLL(path)
        p, i64, i32, u32, u64 = (ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_uint32,
                                 ctypes.c_uint64)
        lib.oracle_mt19937.argtypes = [u32, i64, p]
        lib.oracle_mt19937.restype = None
        lib.oracle_randint.argtypes = [u64, i64, i64, i64, p]
        lib.oracle_randint.restype = i32
        lib.oracle_hash_ids.argtypes = [p, i64, i64, p, i64, p, i64, p, i32, i32, p, p, i64, p]
        lib.oracle_hash_ids.restype = i32
        lib.oracle_hash_prev.argtypes = [p, i64, i64, p, i64, p, i32, i32, p, p, i64, p]
        lib.oracle_hash_prev.restype = i32
        _lib = lib
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


# ------------------------------------------------------------------------------------ layout
def table_layout(num_heads, order_sizes):
    """(table orders, table rows): order-major, head-minor (module.py:65-66)."""
    orders = [n for n in sorted(order_sizes) for _ in range(num_heads)]
    return orders, [int(order_sizes[n]) for n in orders]


def mt19937(seed, n):
    out = np.empty(n, dtype=np.uint32)
    _c().oracle_mt19937(seed, n, _ptr(out))
    return out


def make_mults(seed, n_tables, max_order):
    """torch.randint(1, 2^31-1, (n_tables, max_order), generator=manual_seed(seed)) | 1
    (module.py:94-99), from the C restatement of MT19937 and torch's range mapping."""
    out = np.empty(n_tables * max_order, dtype=np.int64)
    if _c().oracle_randint(seed, 1, PRIME, out.size, _ptr(out)) != 0:
        raise ValueError("seed/range outside what the restatement covers")
    return (out | 1).reshape(n_tables, max_order)


# -------------------------------------------------------------------------------------- hash
def _i64(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.int64))


def hash_ids(input_ids, mults, orders, rows, canon, pad_id, position_ids=None):
    """Row ids [n_tables, B, T] for ids [B, T] (module.py:183-205)."""
    ids = _i64(input_ids)
    if ids.ndim != 2:
        raise ValueError("input_ids must be [batch, seq]")
    B, T = ids.shape
    mults, canon = _i64(mults), _i64(canon)
    pos, pstride = None, 0
    if position_ids is not None:
        pos = _i64(position_ids)
        if pos.ndim == 1:
            pos = pos[None]
        pstride = 0 if pos.shape[0] == 1 else T
        pos = np.ascontiguousarray(np.broadcast_to(pos, (pos.shape[0], T)))
    nt = len(orders)
    out = np.empty((nt, B, T), dtype=np.int64)
    st = _c().oracle_hash_ids(_ptr(ids), B, T, None if pos is None else _ptr(pos), pstride,
                              _ptr(canon), canon.size, _ptr(mults), mults.shape[1], nt,
                              _ptr(np.asarray(orders, dtype=np.int32)), _ptr(_i64(rows)), pad_id,
                              _ptr(out))
    if st != 0:
        raise ValueError("oracle_hash_ids: bad arguments")
    return out


def hash_prev(ids, mults, orders, rows, canon, pad_id):
    """Row ids [n_tables, N] for ids [N, W] of each token and its predecessors (-1 missing)
    (module.py:207-226)."""
    ids, mults, canon = _i64(ids), _i64(mults), _i64(canon)
    N, W = ids.shape
    nt = len(orders)
    out = np.empty((nt, N), dtype=np.int64)
    st = _c().oracle_hash_prev(_ptr(ids), N, W, _ptr(canon), canon.size, _ptr(mults),
                               mults.shape[1], nt, _ptr(np.asarray(orders, dtype=np.int32)),
                               _ptr(_i64(rows)), pad_id, _ptr(out))
    if st != 0:
        raise ValueError("oracle_hash_prev: bad arguments")
    return out


def hash_ids_torch(input_ids, mults, orders, rows, canon, pad_id, position_ids=None):
    """hash_ids as torch-CPU tensor ops, step for step as module.py:183-205 writes them (canon
    after a clamp, left pad with the raw pad id, shifted views, the document-boundary mask, the
    int64 sum of products, then % P % rows): the CPU baseline's hash. Returns int64 [n_tables,
    B, T]."""
    ids = torch.as_tensor(input_ids).long()
    canon = torch.as_tensor(canon).long()
    mults = torch.as_tensor(mults).long()
    ids = canon[ids.clamp(0, canon.numel() - 1)]
    T = ids.shape[-1]
    width = max(orders)
    padded = F.pad(ids, (width - 1, 0), value=pad_id)
    shifted = [padded[:, width - 1 - i: width - 1 - i + T] for i in range(width)]
    if position_ids is not None:
        pos = torch.as_tensor(position_ids).long().expand_as(ids)
        shifted = [s if i == 0 else torch.where(pos >= i, s, torch.full_like(s, pad_id))
                   for i, s in enumerate(shifted)]
    out = []
    for k, n in enumerate(orders):
        x = shifted[0] * mults[k, 0]
        for i in range(1, n):
            x = x + shifted[i] * mults[k, i]
        out.append((x % PRIME) % int(rows[k]))
    return torch.stack(out)


def hash_prev_torch(ids, mults, orders, rows, canon, pad_id):
    """hash_prev as torch-CPU tensor ops, step for step as module.py:207-226 writes them (canon
    after a clamp, missing predecessors (-1) as the raw pad id, the int64 sum of products, then
    % P % rows): the CPU baseline of the serving decode step. Returns int64 [n_tables, N]."""
    ids = torch.as_tensor(ids).long()
    canon = torch.as_tensor(canon).long()
    mults = torch.as_tensor(mults).long()
    merged = canon[ids.clamp(0, canon.numel() - 1)]
    merged = torch.where(ids >= 0, merged, torch.full_like(merged, pad_id))
    out = []
    for k, n in enumerate(orders):
        x = merged[:, 0] * mults[k, 0]
        for i in range(1, n):
            x = x + merged[:, i] * mults[k, i]
        out.append((x % PRIME) % int(rows[k]))
    return torch.stack(out)


def hash_bigint(tokens, mults_row, order, rows):
    """One n-gram row id in Python's arbitrary-precision integers: sum(tok_i * mult_i) % P % rows.
    Exact whenever the int64 sum does not wrap (|tokens| < 2^31)."""
    x = sum(int(tokens[i]) * int(mults_row[i]) for i in range(order))
    return (x % PRIME) % rows


# ------------------------------------------------------------------------------------ gather
def lookup(tables, idx):
    """Concatenated rows [N, n_tables * D] (module.py:146-154, 233); row ids outside a table give
    a zero row, like the masked serving lookup (micro_engram_vllm/tp.py:20-39 at TP=1)."""
    parts = []
    for tab, i in zip(tables, idx):
        i = np.asarray(i, dtype=np.int64).reshape(-1)
        ok = (i >= 0) & (i < tab.shape[0])
        rows = tab[np.where(ok, i, 0)]
        rows[~ok] = 0
        parts.append(rows)
    return np.concatenate(parts, axis=-1)


def lookup_torch(tables, idx):
    """Concatenated rows via torch's CPU embedding, for tables numpy has no dtype for (bf16):
    [F.embedding(idx_k, table_k) for k] then cat (module.py:146-154, 233)."""
    return torch.cat([F.embedding(torch.as_tensor(i).long(), t) for t, i in zip(tables, idx)], dim=-1)


# ------------------------------------------------------------------------------------ inject
def inject(hidden, mem, w_key, w_value, gate="scalar_sqrt", q_scale_delta=None, k_scale_delta=None,
           keep=None, return_alpha=False):
    """torch-CPU restatement of MicroEngram.inject for the scalar gates (module.py:228-261).

    hidden [N, d] (bf16 or fp32); mem [N, M] and w_key/w_value [d, M] in the engram's dtype;
    the scale deltas are the stored q_scale/k_scale parameters (scale - 1, module.py:156-164)."""
    d = hidden.shape[-1]
    # the reference's .float(): bf16 / fp32 -> fp32; float64 inputs (the backward's pinning
    # tests) stay float64
    up = lambda t: t.to(torch.promote_types(t.dtype, torch.float32))
    eps = torch.finfo(torch.float32).eps  # rms_norm's default for the reference's fp32 math
    if gate == "scalar_sqrt":
        q_scale, k_scale = 1 + up(q_scale_delta), 1 + up(k_scale_delta)
        h = F.rms_norm(up(hidden), (d,), weight=q_scale, eps=eps)
        k = F.rms_norm(up(F.linear(mem, w_key)), (d,), weight=k_scale, eps=eps)
    elif gate == "scalar":
        h = F.rms_norm(up(hidden), (d,), eps=eps)
        k = F.rms_norm(up(F.linear(mem, w_key)), (d,), eps=eps)
    else:
        raise ValueError(f"gate {gate!r} is not on this path")
    s = (h * k).sum(-1, keepdim=True) / d ** 0.5
    if gate == "scalar_sqrt":
        s = s.sign() * s.abs().clamp_min(1e-6).sqrt()
    alpha = torch.sigmoid(s)
    out = alpha * up(F.linear(mem, w_value))
    if keep is not None:
        out = out * keep.reshape(*out.shape[:-1], 1).to(out.dtype)
    res = hidden + out.to(hidden.dtype)
    return (res, alpha.reshape(-1)) if return_alpha else res


def inject_backward(grad_out, hidden, mem, w_key, w_value, gate="scalar_sqrt", q_scale_delta=None,
                    k_scale_delta=None, keep=None, stats=None, with_terms=False):
    """Closed-form gradients of inject (module.py:239-261) in float64, from the gradient of its
    output: (d hidden, d K, d V, d q_scale_delta, d k_scale_delta), with K = W_K mem and V = W_V
    mem the key / value Linear outputs (their weight and mem gradients are the plain products
    dK^T mem, dV^T mem, dK W_K + dV W_V). No dtype roundings: the float64 formula itself.

    Per token, with r_h = rsqrt(mean x^2 + eps), r_k = rsqrt(mean K^2 + eps), w = qs * ks,
    sck = sum x w K, s0 = r_h r_k sck / sqrt(d), alpha = sigmoid(s):
      dV = alpha keep g;  d alpha = keep sum g V;  ds = d alpha alpha (1 - alpha)
      ds0 = ds / (2 sqrt|s0|) if |s0| >= 1e-6 else 0 (scalar_sqrt; the scalar gate: ds0 = ds)
      a = ds0 r_h r_k / sqrt(d)
      d hidden = g + a (w K - x r_h^2 sck / d);  dK = a (w x - K r_k^2 sck / d)
      d q_scale_j = ks_j sum_tokens a x_j K_j;  d k_scale_j = qs_j sum_tokens a x_j K_j

    stats: optional [N, 4] (sum x^2, sum K^2, sck, alpha) of a forward that ran elsewhere (the GPU
    forward's row statistics): r_h, r_k, s0 and alpha then come from them instead of from x, K,
    so the closed form is evaluated at that forward's point -- near s0 = 0 the gradient's
    1 / sqrt|s0| factor otherwise turns the forward's own fp32 rounding of s0 into large
    differences. with_terms: also return the scale of each gradient's rounding errors: per
    element the magnitudes its products are made of (|a w K| + |a x r_h^2 sck / d| for d hidden,
    |a w x| + |a K r_k^2 sck / d| for dK, sum_tokens of |a x K| for the scale gradients), each
    token's |a| taken times (1 + sum |g V| / |d alpha|): d alpha is a sum of g V over the row,
    whose rounding is relative to sum |g V|, not to its own (possibly cancelled) size."""
    f = lambda t: t.detach().double()
    x, e, g = f(hidden), f(mem), f(grad_out)
    d = x.shape[-1]
    eps = float(torch.finfo(torch.float32).eps)
    K, V = e @ f(w_key).T, e @ f(w_value).T
    if gate == "scalar_sqrt":
        qs, ks = 1 + f(q_scale_delta), 1 + f(k_scale_delta)
    else:
        qs = ks = torch.ones(d, dtype=torch.float64)
    w = qs * ks
    if stats is None:
        sx2, sk2, sck = (x * x).sum(-1), (K * K).sum(-1), (x * w * K).sum(-1)
    else:
        st = f(stats)
        sx2, sk2, sck = st[:, 0], st[:, 1], st[:, 2]
    rh = 1.0 / torch.sqrt(sx2 / d + eps)
    rk = 1.0 / torch.sqrt(sk2 / d + eps)
    s0 = rh * rk * sck / d ** 0.5
    s = s0.sign() * s0.abs().clamp_min(1e-6).sqrt() if gate == "scalar_sqrt" else s0
    alpha = torch.sigmoid(s) if stats is None else f(stats)[:, 3]
    kf = torch.ones_like(alpha) if keep is None else f(keep.reshape(-1).to(torch.float64))
    dV = (alpha * kf)[:, None] * g
    dalpha = kf * (g * V).sum(-1)
    ds = dalpha * alpha * (1 - alpha)
    if gate == "scalar_sqrt":
        ds0 = torch.where(s0.abs() >= 1e-6, ds / (2 * s0.abs().clamp_min(1e-6).sqrt()), torch.zeros_like(ds))
    else:
        ds0 = ds
    a = ds0 * rh * rk / d ** 0.5
    c2, c3 = (rh * rh * sck / d)[:, None], (rk * rk * sck / d)[:, None]
    dx = g + a[:, None] * (w * K - x * c2)
    dK = a[:, None] * (w * x - K * c3)
    P = (a[:, None] * x * K).sum(0)
    if not with_terms:
        return dx, dK, dV, ks * P, qs * P
    gv = kf * (g * V).abs().sum(-1)
    cond = torch.where(dalpha != 0, 1 + gv / dalpha.abs().clamp_min(1e-300), torch.ones_like(gv))
    aa = (a.abs() * cond)[:, None]
    terms = (aa * ((w * K).abs() + (x * c2).abs()), aa * ((w * x).abs() + (K * c3).abs()),
             (aa * (x * K).abs()).sum(0))
    return dx, dK, dV, ks * P, qs * P, terms


# ------------------------------------------------------------------------------------- dedup
def dedup(keys, grads):
    """(unique keys ascending, inverse, fp32 sums of the grads of each key in index order):
    torch.unique(return_inverse=True) + zeros().index_add_() (rows.py:81, 117-118, 144-146)."""
    keys = np.asarray(keys, dtype=np.int64)
    grads = np.asarray(grads, dtype=np.float32)
    uniq, inv = np.unique(keys, return_inverse=True)
    acc = np.zeros((uniq.size,) + grads.shape[1:], dtype=np.float32)
    np.add.at(acc, inv, grads)  # unbuffered, in index order: ((0 + g_a) + g_b) + ...
    return uniq, inv.astype(np.int64), acc


def dedup_torch(keys, grads):
    """dedup as the reference's torch-CPU ops (rows.py:81, 117-118): torch.unique(return_inverse)
    and zeros().index_add_() of the fp32 gradient rows. The CPU baseline of the sparse update."""
    uniq, inv = torch.unique(torch.as_tensor(keys).long(), return_inverse=True)
    g = torch.as_tensor(grads).float()
    acc = torch.zeros((uniq.numel(),) + tuple(g.shape[1:]), dtype=torch.float32)
    acc.index_add_(0, inv, g)
    return uniq, inv, acc


# -------------------------------------------------------------------------------------- clip
def clip_coef(norm, max_norm):
    """The clipping coefficient of RowTables.clip (rows.py:221-226) from the fp32 norm, in
    fp32 torch-CPU ops as the reference writes them: (max_norm / (norm + 1e-6)).clamp(max=1.0)
    -- the division is Tensor.__rtruediv__, a reciprocal then a product."""
    norm = torch.as_tensor(norm, dtype=torch.float32)
    return (max_norm / (norm + 1e-6)).clamp(max=1.0)


def clip(grads, max_norm):
    """RowTables.clip (rows.py:208-233) on a list of gradients (dense tables' p.grad in any
    float dtype, or sparse_grad fp32 sums): the global norm of all of them, and each scaled in
    place by the coefficient when max_norm > 0 (fp32 sums by the fp32 coefficient, other
    dtypes by the coefficient cast to theirs). Returns the norm as a Python float."""
    sq = torch.zeros((), dtype=torch.float32)
    for g in grads:
        sq += g.float().pow(2).sum()
    norm = sq.sqrt()
    if max_norm and max_norm > 0:
        coef = (max_norm / (norm + 1e-6)).clamp(max=1.0)
        for g in grads:
            g.mul_(coef.to(g.dtype))
    return float(norm)


# ----------------------------------------------------------------------------- random numbers
_PHILOX_M = (np.uint64(0xD2511F53), np.uint64(0xCD9E8D57))
_PHILOX_W = (np.uint32(0x9E3779B9), np.uint32(0xBB67AE85))


def philox4x32_10(ctr, key):
    """Philox4x32 with 10 rounds (Salmon, Moraes, Dror, Shaw, SC'11), vectorised over the
    leading dims: ctr uint32 [..., 4], key uint32 [..., 2] -> uint32 [..., 4]."""
    c = [np.asarray(ctr[..., i], dtype=np.uint32).astype(np.uint64) for i in range(4)]
    k0 = np.asarray(key[..., 0], dtype=np.uint32).copy()
    k1 = np.asarray(key[..., 1], dtype=np.uint32).copy()
    mask = np.uint64(0xFFFFFFFF)
    with np.errstate(over="ignore"):
        for r in range(10):
            p0 = _PHILOX_M[0] * c[0]
            p1 = _PHILOX_M[1] * c[2]
            hi0, lo0 = p0 >> np.uint64(32), p0 & mask
            hi1, lo1 = p1 >> np.uint64(32), p1 & mask
            c = [hi1 ^ c[1] ^ k0.astype(np.uint64), lo1, hi0 ^ c[3] ^ k1.astype(np.uint64), lo0]
            if r < 9:
                k0 = (k0 + _PHILOX_W[0]).astype(np.uint32)
                k1 = (k1 + _PHILOX_W[1]).astype(np.uint32)
    return np.stack([x.astype(np.uint32) for x in c], axis=-1)


def sr_noise(seed, step, table, rows, dim, which):
    """The 16-bit rounding noise of the HIP rowwise-Adam kernel, int32 [len(rows), dim].

    Element (row, col) of array `which` (0: weights, 1: first moment, 2: per-value second
    moment) of table `table` at optimizer step `step` takes 16 bits of Philox4x32-10 with
      counter = (row & 0xffffffff, row >> 32, step, table << 16 | which << 14 | col >> 3)
      key     = (seed & 0xffffffff, seed >> 32)
    word (col >> 1) & 3, half col & 1."""
    rows = np.asarray(rows, dtype=np.int64).astype(np.uint64)
    cols = np.arange(dim, dtype=np.uint64)
    R = rows.size
    ctr = np.empty((R, dim, 4), dtype=np.uint32)
    ctr[..., 0] = (rows & np.uint64(0xFFFFFFFF)).astype(np.uint32)[:, None]
    ctr[..., 1] = (rows >> np.uint64(32)).astype(np.uint32)[:, None]
    ctr[..., 2] = np.uint32(step & 0xFFFFFFFF)
    ctr[..., 3] = ((np.uint64(table) << np.uint64(16)) | (np.uint64(which) << np.uint64(14))
                   | (cols >> np.uint64(3))).astype(np.uint32)[None, :]
    key = np.empty((R, dim, 2), dtype=np.uint32)
    key[..., 0] = np.uint32(seed & 0xFFFFFFFF)
    key[..., 1] = np.uint32((seed >> 32) & 0xFFFFFFFF)
    words = philox4x32_10(ctr, key)
    w = np.take_along_axis(words, ((cols >> np.uint64(1)) & np.uint64(3)).astype(np.int64)[None, :, None]
                           .repeat(R, 0), axis=-1)[..., 0]
    half = (cols & np.uint64(1)).astype(np.uint32)[None, :]
    return ((w >> (np.uint32(16) * half)) & np.uint32(0xFFFF)).astype(np.int32)


def stochastic_bf16(x, noise):
    """fp32 -> bf16 with stochastic rounding (optim.py:33-44): add the 16-bit noise to the fp32
    bit pattern, keep the upper 16 bits; inf/nan pass through. noise: int32 tensor like x."""
    x = x.float().contiguous()
    bits = (x.view(torch.int32) + noise.to(torch.int32)) & -65536
    out = bits.view(torch.float32)
    out = torch.where(torch.isfinite(x), out, x)
    return out.to(torch.bfloat16)


# --------------------------------------------------------------------------------- optimizer
def sparse_adam_step(p, m, v, rows, g, step, lr, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0,
                     stochastic_rounding=True, noise=None):
    """One LazyAdamW step of the sparse-gradient branch, in place (optim.py:65-133, lines 88-97,
    109-132). p [R, D] and m like p (bf16 or fp32), v [R] fp32 (row-wise) or like p; rows int64
    unique ascending with fp32 g [U, D]; step = the step count after this step's increment.
    noise(rows, which) -> int32 [len(rows), D] supplies the bf16 rounding noise (which 0: p,
    1: m, 2: a per-value v). Returns the rows that were updated."""
    beta1, beta2 = betas
    bc1, bc2 = 1 - beta1 ** step, 1 - beta2 ** step
    keep = (g != 0).flatten(1).any(dim=1)
    rows, g = rows[keep], g[keep].float()
    if rows.numel() == 0:
        return rows
    p_ = p.index_select(0, rows).float()
    m_, v_ = m.index_select(0, rows).float(), v.index_select(0, rows).float()
    if weight_decay:
        p_.mul_(1 - lr * weight_decay)
    m_.mul_(beta1).add_(g, alpha=1 - beta1)
    if v_.dim() < g.dim():
        v_.mul_(beta2).add_(g.pow(2).flatten(1).mean(dim=1), alpha=1 - beta2)
        denom = (v_.sqrt() / bc2 ** 0.5).add_(eps).reshape(-1, 1)
    else:
        v_.mul_(beta2).addcmul_(g, g, value=1 - beta2)
        denom = (v_.sqrt() / bc2 ** 0.5).add_(eps)
    p_.addcdiv_(m_, denom, value=-lr / bc1)

    def cast(x, dtype, which):
        if dtype == torch.bfloat16 and stochastic_rounding:
            return stochastic_bf16(x, noise(rows, which))
        return x.to(dtype)

    p.index_copy_(0, rows, cast(p_, p.dtype, 0))
    m.index_copy_(0, rows, cast(m_, m.dtype, 1))
    v.index_copy_(0, rows, cast(v_, v.dtype, 2))
    return rows


# ------------------------------------------------------------------------------ serving ids
def fill_engram_ids(out, input_ids, positions, idx_mapping, query_start_loc, all_token_ids,
                    num_reqs, num_tokens, num_tokens_padded):
    """micro_engram_vllm/ids.py:10-59 restated with explicit loops (numpy, small cases):
    out[t] = (token at t, token at t-1, ...), -1 where there is none. Token t belongs to the
    request whose query_start_loc range holds it; an earlier token in the same chunk (position
    >= the chunk's first position) is read from input_ids[t - k], one before the chunk from the
    request's history row through the reference's lookback index
    j = clamp(chunk_start - 1 - q, 0, max_order - 2) (ids.py:42-55)."""
    out = np.asarray(out)
    max_order = out.shape[1]
    qsl = np.asarray(query_start_loc, dtype=np.int64)
    if num_tokens > 0:
        for r in range(num_reqs):
            b, e = int(qsl[r]), int(qsl[r + 1])
            start = int(positions[min(b, num_tokens - 1)])
            hist = np.asarray(all_token_ids)[int(idx_mapping[r])]
            look = [int(hist[start - 1 - j]) if start - 1 - j >= 0 else -1 for j in range(max_order - 1)]
            for t in range(b, min(e, num_tokens)):
                p = int(positions[t])
                out[t, 0] = input_ids[t]
                for k in range(1, max_order):
                    q = p - k
                    if q >= start:
                        out[t, k] = input_ids[max(t - k, 0)]
                    else:
                        out[t, k] = look[min(max(start - 1 - q, 0), max_order - 2)]
    out[num_tokens:num_tokens_padded] = -1
    return out


def mask_media(ids, media_ids):
    """micro_engram_vllm/ids.py:62-70: media placeholder ids become -1 (missing history);
    keep[t] is False where the token itself (column 0) is a media placeholder."""
    ids = np.asarray(ids)
    is_media = np.isin(ids, np.asarray(media_ids))
    return np.where(is_media, -1, ids).astype(ids.dtype), ~is_media[:, 0]
