"""BlockMask-style layout of the SCOPE pointer mask.

``ScopeBlockMask`` carries the compact rows the kernels use — ``kv_num_blocks
[1,H,QB]`` and ``kv_indices [1,H,QB,MAXKV]`` (unique blocks ascending, then
the duplicates, exactly as ``model/attn_bias.py:825-837`` packs them) — plus
the document information the mask_mod needs.  ``to_torch_blockmask()``
exports the reference's NB-wide layout (``model/attn_bias.py:851-873``) as a
real ``torch.nn.attention.flex_attention.BlockMask`` for interoperability.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import ops


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
            self._q_lists = ops.transpose_blocks(self.kv_num_blocks[0], self.kv_indices[0], self.num_blocks)
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
        """torch ``BlockMask`` equal to the reference's (full_* = zeros)."""
        from torch.nn.attention.flex_attention import BlockMask

        kv_num = self.kv_num_blocks.contiguous()
        kv_idx = self.kv_indices_export().contiguous()
        return BlockMask.from_kv_blocks(kv_num, kv_idx, torch.zeros_like(kv_num), torch.zeros_like(kv_idx),
                                        BLOCK_SIZE=self.BLOCK_SIZE, mask_mod=self.document_causal())

    def active_tiles(self) -> torch.Tensor:
        """N_act = Σ kv_num_blocks (device scalar, no host sync)."""
        return self.kv_num_blocks.sum()
