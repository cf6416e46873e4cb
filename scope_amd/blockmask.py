"""BlockMask-style layout of the SCOPE block masks.

``ScopeBlockMask`` carries the compact rows the kernels use — ``kv_num_blocks
[1,H,QB]`` and ``kv_indices [1,H,QB,MAXKV]`` — plus the document information
the mask_mod needs.  Two producers fill it:

* the pointer mask (unique blocks ascending, then the duplicates, exactly as
  ``model/attn_bias.py:825-837`` packs them);
* ``create_blockmasks``, the long / short sliding-window masks of the layers
  without the pointer mask (``scoped_medium.py:535-576``): the union of the
  window's full and partial blocks.  The attention kernels decide per tile
  whether the causal / document mask can be skipped, which covers the full
  blocks' fast path.

``to_torch_blockmask()`` exports the reference's NB-wide layout
(``model/attn_bias.py:851-873``, or the partial / full lists of
``scoped_medium.py:566-573``) as a real
``torch.nn.attention.flex_attention.BlockMask`` for interoperability.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import library, ops


@dataclass
class ScopeBlockMask:
    kv_num_blocks: torch.Tensor  # [1, H, QB] int32
    kv_indices: torch.Tensor     # [1, H, QB, MAXKV] int32 (compact)
    BLOCK_SIZE: int
    docs: torch.Tensor           # [T] int32 document ids
    ds_tok_end: torch.Tensor     # [QB] int32 doc start token of each block's last token
    ds_ptr: torch.Tensor | None = None
    ds_local: torch.Tensor | None = None
    extras: dict = field(default_factory=dict)  # radius / centre (reference mode), picks / logits (block scoring)
    _q_lists: tuple | None = field(default=None, repr=False)
    # validate the lists on construction (ops.check_lists: 0 <= kv_num <= MAXKV
    # distinct key blocks in [0, NB), each <= its q-block; RuntimeError
    # otherwise); the library's own builders, whose kernels guarantee that,
    # pass False
    check: bool = field(default=True, repr=False)

    def __post_init__(self):
        if self.kv_num_blocks.shape[-1] * self.BLOCK_SIZE != self.docs.numel():
            raise RuntimeError(f"ScopeBlockMask: {self.kv_num_blocks.shape[-1]} q-blocks of {self.BLOCK_SIZE} do not "
                               f"cover the {self.docs.numel()} document ids")
        if self.check:
            ops.check_lists(self.kv_num_blocks, self.kv_indices, self.num_blocks, who="ScopeBlockMask")

    @property
    def seq_len(self) -> int:
        return int(self.docs.numel())

    @property
    def num_blocks(self) -> int:
        return self.seq_len // self.BLOCK_SIZE

    @property
    def num_heads(self) -> int:
        return int(self.kv_num_blocks.shape[-2])

    @property
    def maxkv(self) -> int:
        return int(self.kv_indices.shape[-1])

    @property
    def shape(self) -> tuple[int, int, int, int]:
        return (1, self.num_heads, self.seq_len, self.seq_len)

    def q_lists(self) -> tuple[torch.Tensor, torch.Tensor]:
        """Transposed lists (CSR): q_off [H, NB+1], q_list [H, QB*MAXKV]."""
        if self._q_lists is None:
            self._q_lists = library.transpose_blocks(self.kv_num_blocks[0], self.kv_indices[0], self.num_blocks)
        return self._q_lists

    def kv_indices_export(self) -> torch.Tensor:
        """NB-wide kv_indices (model/attn_bias.py:851-860): truncate when
        MAXKV >= NB, else pad the tail with the first packed entry."""
        nb, mk = self.num_blocks, self.maxkv
        if mk >= nb:
            return self.kv_indices[..., :nb].contiguous()
        out = self.kv_indices[..., :1].expand(*self.kv_indices.shape[:-1], nb).clone()
        out[..., :mk] = self.kv_indices
        return out

    def document_causal(self):
        docs = self.docs

        def document_causal(b, h, q_idx, kv_idx):  # model/attn_bias.py:674-679
            q = q_idx.to(torch.long)
            k = kv_idx.to(torch.long)
            return (q >= k) & (docs[q] == docs[k])

        return document_causal

    def to_torch_blockmask(self):
        """torch ``BlockMask`` equal to the reference's: the pointer mask with
        full_* = zeros, or a sliding-window mask with its partial / full lists
        (built with ``create_blockmasks(..., export=True)``)."""
        from torch.nn.attention.flex_attention import BlockMask

        swa = self.extras.get("swa")
        if swa is not None:
            if swa.get("partial_idx") is None:
                raise RuntimeError("to_torch_blockmask: build the mask with create_blockmasks(..., export=True)")
            r4 = lambda t: t.reshape(1, 1, *t.shape).contiguous()
            return BlockMask.from_kv_blocks(r4(swa["kv_num_blocks"]), r4(swa["partial_idx"]),
                                            r4(swa["full_kv_num_blocks"]), r4(swa["full_idx"]),
                                            BLOCK_SIZE=self.BLOCK_SIZE, mask_mod=self.document_causal())
        kv_num = self.kv_num_blocks.contiguous()
        kv_idx = self.kv_indices_export().contiguous()
        return BlockMask.from_kv_blocks(kv_num, kv_idx, torch.zeros_like(kv_num), torch.zeros_like(kv_idx),
                                        BLOCK_SIZE=self.BLOCK_SIZE, mask_mod=self.document_causal())

    def active_tiles(self) -> torch.Tensor:
        """N_act = Σ kv_num_blocks (device scalar, no host sync)."""
        return self.kv_num_blocks.sum()


def create_blockmasks(input_seq: torch.Tensor | None, sliding_window_num_blocks, docs: torch.Tensor | None = None, *,
                      num_heads: int = 1, block_size: int = 128, export: bool = False):
    """(long, short) sliding-window masks of ``GPT.create_blockmasks``
    (scoped_medium.py:535-576) for ``num_heads`` heads.

    ``docs`` defaults to ``cumsum(input_seq == 50256)`` (:537-538); the
    window is W blocks for the long mask and W // 2 for the short one.  With
    ``export`` the reference-format partial / full lists are kept for
    ``to_torch_blockmask()``."""
    if docs is None:
        if input_seq is None:
            raise RuntimeError("create_blockmasks: give input_seq or docs")
        docs = (input_seq.reshape(-1) == 50256).cumsum(0)
    docs = docs.reshape(-1).to(torch.int32).contiguous()
    T = docs.numel()
    if T % block_size:
        raise RuntimeError(f"create_blockmasks: T={T} is not a multiple of {block_size}")
    W = int(sliding_window_num_blocks.item() if torch.is_tensor(sliding_window_num_blocks)
            else sliding_window_num_blocks)
    r = ops.swa_blockmask(docs, block_size, W, export=export)
    _, _, ds_tok_end = ops.doc_starts(docs, block_size)
    out = []
    for i, name in enumerate(("long", "short")):
        kv_num, kv_idx = r[name]
        swa = dict(kv_num_blocks=r["counts"][2 + 2 * i], full_kv_num_blocks=r["counts"][3 + 2 * i],
                   partial_idx=r["partial_idx"], full_idx=r["full_idx"], window_blocks=W if i == 0 else W // 2)
        out.append(ScopeBlockMask(
            kv_num_blocks=kv_num.expand(num_heads, -1).reshape(1, num_heads, -1).contiguous(),
            kv_indices=kv_idx.expand(num_heads, -1, -1).reshape(1, num_heads, *kv_idx.shape).contiguous(),
            BLOCK_SIZE=block_size, docs=docs, ds_tok_end=ds_tok_end, extras=dict(swa=swa), check=False))
    return out[0], out[1]
