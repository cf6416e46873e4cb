"""CPU oracle: pointer-driven block selection and the BlockMask-style layout.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference mode restates ``model/attn_bias.py:623-873``
(``SpectralBias.build_pointer_blockmask``) step by step in numpy with the same
fp32 arithmetic.  Block-scoring mode is the block-mean q·k pointer selection
(a specification of this project, not present in the reference); its
definition lives here and in ``scope_amd/csrc/pointer.hip``.

Parity pins (tests/test_oracle_pointer.py):

* ``doc_start_blocks``        – golden vectors from the reference + brute force.
* ``radius_alloc_pi``         – golden vectors; Σr = budget_rem invariant; M=1.
* ``pointer_mask_reference``  – golden vectors (10 configurations covering pi /
                                fixed radius, Gumbel, resets, doc clamp off,
                                p=0, disabled, export truncation, overrides).
* ``pack_sorted_unique``      – golden vectors + brute-force set union.
* ``transpose_blocks``        – torch ``BlockMask`` (library) ``q_indices``.
* ``pointer_select_blockscore`` – brute force over all candidate subsets on
                                tiny inputs; invariants.
* ``gumbel_from_u``           – closed form.
* ``counter_uniform``         – fixed known-answer values (integer hash).
"""
from __future__ import annotations

import numpy as np

F32 = np.float32


# --------------------------------------------------------------------------
# doc starts  (model/attn_bias.py:688-709)
# --------------------------------------------------------------------------
def doc_start_token(docs: np.ndarray) -> np.ndarray:
    """Most recent change point ≤ t (model/attn_bias.py:688-691)."""
    docs = np.asarray(docs)
    T = docs.shape[0]
    change = np.ones(T, dtype=bool)
    change[1:] = docs[1:] != docs[:-1]
    idx = np.arange(T, dtype=np.int64)
    return np.maximum.accumulate(np.where(change, idx, 0))


def doc_start_blocks(docs, bs: int, *, doc_clamp: bool = True, reset_active: bool = False,
                     reset_len: int = 0):
    """Per q-block doc-start blocks, as the pointer mask uses them.

    Returns ``(ds_ptr, ds_local, ds_tok_end)``:

    * ``ds_ptr[qb]``   doc start block of the representative (last) token,
                       ``model/attn_bias.py:693``, clamped by resets ``:703-709``;
    * ``ds_local[qb]`` doc start block of the first token of the block, ``:696-697``;
    * ``ds_tok_end[qb]`` doc start *token* of the block's last token, ignoring
      ``doc_clamp`` and resets: the attention kernel uses it to classify a tile
      as unmasked (no document change between the key tile and the query rows).
    """
    dst = doc_start_token(docs)
    T = dst.shape[0]
    NB = T // bs
    qb = np.arange(NB, dtype=np.int64)
    t_rep = (qb + 1) * bs - 1
    first = qb * bs
    tok_end = dst[t_rep].astype(np.int32)
    ds_ptr = (dst[t_rep] // bs).astype(np.int64)
    ds_local = (dst[first] // bs).astype(np.int64)
    if not doc_clamp:
        ds_ptr = np.zeros_like(ds_ptr)
        ds_local = np.zeros_like(ds_local)
    if reset_active and reset_len > 0:
        seg_ptr = ((t_rep // reset_len) * reset_len) // bs
        seg_loc = ((first // reset_len) * reset_len) // bs
        ds_ptr = np.maximum(ds_ptr, seg_ptr)
        ds_local = np.maximum(ds_local, seg_loc)
    return ds_ptr.astype(np.int32), ds_local.astype(np.int32), tok_end


# --------------------------------------------------------------------------
# representatives  (model/attn_bias.py:713-719)
# --------------------------------------------------------------------------
def representatives(x: np.ndarray, bs: int, rep_mode: str) -> np.ndarray:
    """x: [H,T,M] fp32 -> [H,QB,M] at t_rep=(qb+1)·bs-1 ("last") or the block
    mean ("mean"; fp32 result of an fp64 sum, so it can differ from torch's
    fp32 reduction in the last bit)."""
    H, T, M = x.shape
    NB = T // bs
    if rep_mode == "last":
        t_rep = (np.arange(NB) + 1) * bs - 1
        return np.ascontiguousarray(x[:, t_rep, :]).astype(F32)
    return x.reshape(H, NB, bs, M).astype(np.float64).mean(axis=2).astype(F32)


def sigmoid32(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=F32)
    return (F32(1.0) / (F32(1.0) + np.exp(-x))).astype(F32)


# --------------------------------------------------------------------------
# radius allocation  (model/attn_bias.py:721-761)
# --------------------------------------------------------------------------
def budget_rem_blocks(*, M: int, local_blocks: int, ptr_half_blocks: int, budget_blocks: int,
                      budget_is_total: bool) -> int:
    """Integer half-budget ``budget_rem`` (model/attn_bias.py:724-734)."""
    budget_val = max(0, int(budget_blocks))
    if budget_is_total:
        cap = int(local_blocks + M + 2 * M * int(ptr_half_blocks))
        total = min(budget_val, cap)
        extra = max(total - int(local_blocks) - int(M), 0)
    else:
        extra = budget_val
    rem = extra // 2
    return min(rem, M * int(ptr_half_blocks))


def radius_alloc_pi(budget_rep: np.ndarray, *, budget_rem: int, temp: float, p: int) -> np.ndarray:
    """Stick-breaking + largest remainder (model/attn_bias.py:735-758).

    Ties in the fractional parts are broken toward the lower peak index (the
    reference's ``argsort`` is not stable, so its tie order is unspecified)."""
    H, QB, M = budget_rep.shape
    if budget_rem <= 0:
        return np.zeros((H, QB, M), dtype=np.int32)
    t = F32(max(float(temp), 1e-6))
    u = (budget_rep.astype(F32) / t).astype(F32)
    rem = np.full((H, QB), F32(budget_rem), dtype=F32)
    alloc = np.zeros((H, QB, M), dtype=F32)
    for m in range(M - 1):
        v = sigmoid32(u[..., m])
        b = (v * rem).astype(F32)
        alloc[..., m] = b
        rem = (rem - b).astype(F32)
    alloc[..., M - 1] = rem
    fl = np.floor(alloc).astype(F32)
    frac = (alloc - fl).astype(F32)
    floor_sum = fl.astype(np.int64).sum(axis=-1)
    rem_int = np.clip(budget_rem - floor_sum, 0, M)
    order = np.argsort(-frac, axis=-1, kind="stable")
    rank = np.argsort(order, axis=-1, kind="stable")
    add = rank < rem_int[..., None]
    extra = fl.astype(np.int64) + add
    return np.clip(extra, 0, p).astype(np.int32)


def gumbel_from_u(u: np.ndarray, eps: float = 1e-9) -> np.ndarray:
    """g = -log(-log(u+eps)+eps) in fp32 (model/attn_bias.py:771)."""
    e = F32(eps)
    u = np.asarray(u, dtype=F32)
    return (-np.log((-np.log((u + e).astype(F32))).astype(F32) + e)).astype(F32)


def gumbel_peak_mask(budget_rep: np.ndarray, u: np.ndarray, *, k: int, tau: float, eps: float) -> np.ndarray:
    """Top-k peaks by budget/τ + g (model/attn_bias.py:763-777); ties → lower index."""
    H, QB, M = budget_rep.shape
    t = F32(max(float(tau), 1e-6))
    scores = ((budget_rep.astype(F32) / t).astype(F32) + gumbel_from_u(u, eps)).astype(F32)
    order = np.argsort(-scores, axis=-1, kind="stable")
    mask = np.zeros((H, QB, M), dtype=bool)
    np.put_along_axis(mask, order[..., :k], True, axis=-1)
    return mask


# --------------------------------------------------------------------------
# sort / dedupe / pack  (model/attn_bias.py:825-837) and export (:851-860)
# --------------------------------------------------------------------------
def pack_sorted_unique(kv_blocks: np.ndarray):
    """[..., MAXKV] -> (kv_num [...], packed [..., MAXKV]).

    ``packed`` holds the unique blocks ascending, then the duplicates
    ascending, exactly like the reference's two-key sort."""
    s = np.sort(kv_blocks, axis=-1)
    keep = np.ones_like(s, dtype=bool)
    keep[..., 1:] = s[..., 1:] != s[..., :-1]
    kv_num = keep.sum(axis=-1).astype(np.int32)
    order = np.argsort(~keep, axis=-1, kind="stable")  # keeps first (ascending), dups after (ascending)
    packed = np.take_along_axis(s, order, axis=-1).astype(np.int32)
    return kv_num, packed


def export_nb_wide(packed: np.ndarray, NB: int) -> np.ndarray:
    """NB-wide kv_indices for ``BlockMask.from_kv_blocks`` (model/attn_bias.py:851-860)."""
    maxkv = packed.shape[-1]
    if maxkv >= NB:
        return np.ascontiguousarray(packed[..., :NB]).astype(np.int32)
    out = np.empty(packed.shape[:-1] + (NB,), dtype=np.int32)
    out[..., :maxkv] = packed
    out[..., maxkv:] = packed[..., :1]
    return out


def transpose_blocks(kv_num: np.ndarray, kv_idx: np.ndarray, NB: int):
    """q lists: for each kv block, the q-blocks listing it, ascending.

    Returns CSR per head: ``q_off [H, NB+1]`` and ``q_list [H, total]``, plus
    the dense ``q_num [H, NB]``.  Equals torch's ``_transpose_ordered``
    (dense -> transpose -> stable argsort) restricted to the first ``q_num``
    entries of each row."""
    H, QB = kv_num.shape
    q_num = np.zeros((H, NB), dtype=np.int32)
    lists = [[[] for _ in range(NB)] for _ in range(H)]
    for h in range(H):
        for qb in range(QB):
            for i in range(int(kv_num[h, qb])):
                kb = int(kv_idx[h, qb, i])
                lists[h][kb].append(qb)
                q_num[h, kb] += 1
    q_off = np.zeros((H, NB + 1), dtype=np.int32)
    q_off[:, 1:] = np.cumsum(q_num, axis=1)
    total = int(q_off[:, -1].max()) if H else 0
    q_list = np.full((H, max(total, 1)), -1, dtype=np.int32)
    for h in range(H):
        flat = [qb for kb in range(NB) for qb in sorted(lists[h][kb])]
        q_list[h, : len(flat)] = flat
    return q_num, q_off, q_list


def transpose_dense_export(kv_num: np.ndarray, kv_idx: np.ndarray, NB: int):
    """torch ``_transpose_ordered`` semantics: [H, NB] counts and [H, NB, QB]
    rows listing users ascending, then non-users ascending."""
    H, QB = kv_num.shape
    dense = np.zeros((H, QB, NB), dtype=np.int32)
    for h in range(H):
        for qb in range(QB):
            for i in range(int(kv_num[h, qb])):
                dense[h, qb, int(kv_idx[h, qb, i])] = 1
    dT = np.transpose(dense, (0, 2, 1))
    q_num = dT.sum(-1).astype(np.int32)
    q_idx = np.argsort(-dT, axis=-1, kind="stable").astype(np.int32)
    return q_num, q_idx


# --------------------------------------------------------------------------
# reference mode  (model/attn_bias.py:623-873)
# --------------------------------------------------------------------------
def pointer_mask_reference(delta_rep: np.ndarray, budget_rep: np.ndarray, docs: np.ndarray, *,
                           bs: int, M: int, local_blocks: int, ptr_half_blocks: int,
                           global_blocks_cfg: int, global_active: int, budget_blocks: int,
                           budget_is_total: bool, budget_temp: float, radius_mode: str,
                           doc_clamp: bool, mask_active: bool, half_active: int,
                           reset_active: bool = False, reset_len: int = 0,
                           gumbel_active: bool = False, gumbel_k: int = 0, gumbel_tau: float = 1.0,
                           gumbel_u: np.ndarray | None = None, eps: float = 1e-9) -> dict:
    """Reference-mode pointer mask from representatives.

    ``delta_rep``/``budget_rep`` are [H,QB,M] fp32 (see ``representatives``).
    ``local_blocks``/``ptr_half_blocks``/``budget_blocks`` are the values
    after the call-site overrides; ``global_active`` is the active global count
    (``global_blocks`` argument or the scheduled buffer).  ``gumbel_active``
    folds ``training and gumbel_topk and p > 0 and k < M``.
    """
    H, QB, _ = delta_rep.shape
    T = docs.shape[0]
    NB = T // bs
    assert QB == NB
    local_blocks = min(max(1, int(local_blocks)), NB)
    p = max(0, int(ptr_half_blocks))
    ds_ptr, ds_local, _ = doc_start_blocks(docs, bs, doc_clamp=doc_clamp,
                                           reset_active=reset_active, reset_len=reset_len)
    qb = np.arange(NB, dtype=np.int64)
    t_rep = (qb + 1) * bs - 1

    if radius_mode == "fixed":
        r = np.full((H, NB, M), int(half_active), dtype=np.int64)
    else:
        rem = budget_rem_blocks(M=M, local_blocks=local_blocks, ptr_half_blocks=p,
                                budget_blocks=budget_blocks, budget_is_total=budget_is_total)
        r = radius_alloc_pi(budget_rep, budget_rem=rem, temp=budget_temp, p=p).astype(np.int64)
    r = np.minimum(r, int(half_active))
    if not mask_active:
        r = np.zeros_like(r)
    if gumbel_active:
        keep = gumbel_peak_mask(budget_rep, gumbel_u, k=gumbel_k, tau=gumbel_tau, eps=eps)
        r = np.where(keep, r, 0)

    key = (t_rep[None, :, None].astype(F32) - delta_rep.astype(F32)).astype(F32)
    key = np.maximum(key, F32(0.0))
    centre = key.astype(np.int64) // bs
    centre = np.minimum(centre, qb[None, :, None])
    if not mask_active:
        centre = np.broadcast_to(qb[None, :, None], (H, NB, M)).copy()
    centre = np.maximum(centre, ds_ptr[None, :, None].astype(np.int64))

    pieces = []
    offs_local = np.arange(local_blocks)
    local = np.maximum(qb[:, None] - offs_local[None, :], 0)
    local = np.maximum(local, ds_local[:, None])
    pieces.append(np.broadcast_to(local[None], (H, NB, local_blocks)))
    if p > 0:
        offs = np.arange(-p, p + 1)
        active = np.abs(offs)[None, None, None, :] <= r[..., None]
        ptr = centre[..., None] + offs[None, None, None, :]
        ptr = np.clip(ptr, 0, NB - 1)
        ptr = np.minimum(ptr, qb[None, :, None, None])
        ptr = np.maximum(ptr, ds_ptr[None, :, None, None])
        ptr = np.where(active, ptr, centre[..., None])
        pieces.append(ptr.reshape(H, NB, M * (2 * p + 1)))
    else:
        pieces.append(centre)
    gmax = min(int(global_blocks_cfg), NB)
    if gmax > 0:
        g = np.arange(gmax)
        gl = np.minimum(ds_ptr[:, None].astype(np.int64) + g[None, :], qb[:, None])
        ga = int(np.clip(global_active, 0, gmax))
        gl = np.where((g < ga)[None, :], gl, qb[:, None])
        pieces.append(np.broadcast_to(gl[None], (H, NB, gmax)))
    kv_blocks = np.concatenate([np.asarray(x, dtype=np.int64) for x in pieces], axis=-1).astype(np.int32)
    kv_num, packed = pack_sorted_unique(kv_blocks)
    return dict(kv_num=kv_num, packed=packed, radius=r.astype(np.int32), centre=centre.astype(np.int32),
                ds_ptr=ds_ptr, ds_local=ds_local, maxkv=kv_blocks.shape[-1])


# --------------------------------------------------------------------------
# block-scoring mode (this project's specification)
# --------------------------------------------------------------------------
def _mix32(x: np.ndarray) -> np.ndarray:
    """32-bit avalanche (the lowbias32 integer hash: xor-shift 16, multiply by
    0x7feb352d, xor-shift 15, multiply by 0x846ca68b, xor-shift 16)."""
    x = x.astype(np.uint32)
    x ^= x >> np.uint32(16)
    x = (x * np.uint32(0x7FEB352D)).astype(np.uint32)
    x ^= x >> np.uint32(15)
    x = (x * np.uint32(0x846CA68B)).astype(np.uint32)
    x ^= x >> np.uint32(16)
    return x


def counter_uniform(seed: int, h: np.ndarray, qb: np.ndarray, kb: np.ndarray) -> np.ndarray:
    """Counter-based uniform in [0,1) for the in-kernel Gumbel draw:
    u = (hash(seed, h, qb, kb) >> 8) · 2^-24, with
    hash = mix(mix(mix(mix(seed_lo ^ mix(seed_hi)) ^ h) ^ qb) ^ kb) and each
    step ``mix(a ^ (b + 0x9e3779b9·(step+1)))``."""
    s = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
    lo = np.uint32(int(s) & 0xFFFFFFFF)
    hi = np.uint32(int(s) >> 32)
    with np.errstate(over="ignore"):
        x = _mix32(np.asarray(lo ^ _mix32(np.asarray(hi, np.uint32)), np.uint32))
        for step, v in enumerate((h, qb, kb)):
            k = np.uint32((0x9E3779B9 * (step + 1)) & 0xFFFFFFFF)
            x = _mix32(x ^ (np.asarray(v).astype(np.uint32) + k).astype(np.uint32))
    return ((x >> np.uint32(8)).astype(np.float64) * (1.0 / 16777216.0)).astype(F32)


def block_means(x: np.ndarray, bs: int) -> np.ndarray:
    """[H,T,D] -> [H,NB,D] block means in fp64."""
    H, T, D = x.shape
    return x.reshape(H, T // bs, bs, D).astype(np.float64).mean(axis=2)


def pointer_logits(qbar: np.ndarray, kbar: np.ndarray, *, logit_scale: float,
                   prior: np.ndarray | None = None) -> np.ndarray:
    """logit[h,qb,kb] = logit_scale · q̄·k̄ + prior[h, qb-kb] for kb ≤ qb (fp64)."""
    H, NB, D = qbar.shape
    lg = logit_scale * np.einsum("hqd,hkd->hqk", qbar, kbar)
    if prior is not None:
        pr = np.broadcast_to(np.asarray(prior, np.float64).reshape(-1, NB), (H, NB))
        d = np.arange(NB)[:, None] - np.arange(NB)[None, :]
        lg = lg + np.where(d >= 0, pr[:, np.clip(d, 0, NB - 1)], 0.0)
    return lg


def window_and_global(qb: int, ds_ptr: int, ds_local: int, W: int, G: int, NB: int):
    win = [max(max(qb - o, 0), ds_local) for o in range(min(W, NB))]
    glb = [min(ds_ptr + g, qb) for g in range(min(G, NB))]
    return win, glb


def pointer_select_blockscore(logits: np.ndarray, docs: np.ndarray, *, bs: int, window: int,
                              n_global: int, budget: int, temp: float = 1.0,
                              gumbel: np.ndarray | None = None, doc_clamp: bool = True,
                              rows=None) -> dict:
    """Block-scoring selection from fp32 logits [H,QB,NB].

    Per (h, qb):
      window  = {max(max(qb-o,0), ds_local) : o < W}
      global  = {min(ds_ptr+g, qb) : g < G}
      cand    = {kb : ds_ptr ≤ kb ≤ qb} \\ (window ∪ global)
      z(kb)   = logits/τ (+ g(kb) if Gumbel noise is given), fp32
      picks   = top-``budget`` of cand by z, ties → lower kb; short lists are
                padded with qb (removed again by the dedupe)
      list    = sort-dedupe-pack(window ++ picks ++ global)
    ``gumbel`` is the transformed noise g [H,QB,NB] (fp32), or None.
    ``rows``: compute only these q-blocks (the other rows of the result are
    left as for an empty selection), for long sequences in tests."""
    H, QB, NB = logits.shape
    ds_ptr, ds_local, _ = doc_start_blocks(docs, bs, doc_clamp=doc_clamp)
    t = F32(max(float(temp), 1e-6))
    W = min(window, NB)
    G = min(n_global, NB)
    maxkv = W + budget + G
    raw = np.zeros((H, QB, maxkv), dtype=np.int32)
    picks = np.full((H, QB, budget), -1, dtype=np.int32)
    for h in range(H):
        for qb in (range(QB) if rows is None else rows):
            win, glb = window_and_global(qb, int(ds_ptr[qb]), int(ds_local[qb]), W, G, NB)
            excl = set(win) | set(glb)
            cand = [kb for kb in range(int(ds_ptr[qb]), qb + 1) if kb not in excl]
            z = (logits[h, qb, cand].astype(F32) / t).astype(F32)
            if gumbel is not None:
                z = (z + gumbel[h, qb, cand].astype(F32)).astype(F32)
            order = sorted(range(len(cand)), key=lambda i: (-float(z[i]), cand[i]))
            sel = [cand[i] for i in order[:budget]]
            picks[h, qb, : len(sel)] = sel
            sel = sel + [qb] * (budget - len(sel))
            raw[h, qb] = np.asarray(win + sel + glb, dtype=np.int32)
    kv_num, packed = pack_sorted_unique(raw)
    return dict(kv_num=kv_num, packed=packed, picks=picks, ds_ptr=ds_ptr, ds_local=ds_local, maxkv=maxkv)


def soft_pair_bias(logits: np.ndarray, kv_num: np.ndarray, kv_idx: np.ndarray, picks: np.ndarray, *,
                   soft_temp: float) -> np.ndarray:
    """Soft top-k weights of the pointer picks as an additive score bias per
    list entry (a specification of this project; the reference selects under
    ``torch.no_grad``, model/attn_bias.py:623).

        b[h,qb,e] = log σ(logit[h,qb,kb]/τ_w)   for e < kv_num and kb = kv_idx[h,qb,e] a pick
        b[h,qb,e] = 0                           for window, global and padding entries

    ``logits`` are the noise-free block-scoring logits [H,QB,NB] (fp64)."""
    H, QB, L = kv_idx.shape
    out = np.zeros((H, QB, L), dtype=np.float64)
    t = float(soft_temp)
    for h in range(H):
        for qb in range(QB):
            pk = set(int(x) for x in picks[h, qb] if x >= 0)
            for e in range(int(kv_num[h, qb])):
                kb = int(kv_idx[h, qb, e])
                if kb in pk:
                    x = float(logits[h, qb, kb]) / t
                    out[h, qb, e] = -np.logaddexp(0.0, -x)  # log σ(x)
    return out
