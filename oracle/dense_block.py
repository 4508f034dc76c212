"""The reference's MultiAnchorRelationBlock structure as a dense torch module
(src/relation_lm/models/multi_relation_blocks.py:21-187) -- TEST
INFRASTRUCTURE ONLY (see oracle/__init__.py): the independent formulation the
oracle and the routed HIP block are checked against (dense causal selection: iterative distinct-anchor argmax with
F.one_hot masks, torch.topk over the all-anchor-masked partner scores)."""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn


class DenseBlock(nn.Module):
    """The reference block's structure in float64 (dense causal selection)."""

    def __init__(self, d, g, r, slots, k, ff_mult=2):
        super().__init__()
        self.h, self.k, self.g = slots, k, g
        self.input_norm = nn.LayerNorm(d)
        self.anchor_query = nn.Linear(d, slots * g, bias=False)
        self.anchor_key = nn.Linear(d, slots * g, bias=False)
        self.partner_query = nn.ModuleList(nn.Linear(2 * d, g, bias=False) for _ in range(slots))
        self.partner_key = nn.Linear(d, slots * g, bias=False)
        self.operand = nn.Linear(d, r, bias=False)
        self.relation_mlp = nn.Sequential(nn.Linear(4 * r, ff_mult * d), nn.GELU(),
                                          nn.Linear(ff_mult * d, d), nn.LayerNorm(d))
        self.slot_mix_logits = nn.Parameter(torch.randn(slots))
        self.residual_gate = nn.Parameter(torch.tensor(0.3))

    @staticmethod
    def gather(source, index):
        shape = (source.size(0),) + (1,) * (index.ndim - 1)
        batch = torch.arange(source.size(0)).view(shape)
        return source[batch.expand_as(index), index]

    def forward(self, hidden, memory):
        b, t, _ = hidden.shape
        h, g, kc = self.h, self.g, self.k
        x = self.input_norm(hidden)
        causal = torch.triu(torch.ones(t, t, dtype=torch.bool), diagonal=1)
        q = self.anchor_query(x).view(b, t, h, g)
        kk = self.anchor_key(memory).view(b, t, h, g)
        score = torch.einsum("bthd,bshd->bhts", q, kk) * g ** -0.5
        score = score.masked_fill(causal[None, None], -torch.inf)
        active = torch.arange(h)[None, :] <= torch.arange(t)[:, None]
        selected = []
        for s in range(h):
            ss = score[:, s]
            if selected:
                used = F.one_hot(torch.stack(selected, -1), num_classes=t).any(dim=-2)
                ss = ss.masked_fill(used, -torch.inf)
            idx = ss.argmax(dim=-1)
            selected.append(torch.where(active[:, s][None].expand(b, -1), idx, torch.zeros_like(idx)))
        anchor_index = torch.stack(selected, -1)
        anchor = self.gather(memory, anchor_index) * active[None, :, :, None].to(memory.dtype)
        pin = torch.cat((x[:, :, None].expand(-1, -1, h, -1), anchor), -1)
        pq = torch.stack([layer(pin[:, :, s]) for s, layer in enumerate(self.partner_query)], 2)
        pk = self.partner_key(memory).view(b, t, h, g)
        ps = torch.einsum("bthd,bshd->bhts", pq, pk) * g ** -0.5
        ps = ps.masked_fill(causal[None, None], -torch.inf)
        anchor_active = active[None].expand(b, -1, -1)
        all_anchor = (F.one_hot(anchor_index, num_classes=t) & anchor_active.unsqueeze(-1)).any(-2)
        ps = ps.masked_fill(all_anchor[:, None].expand(-1, h, -1, -1), -torch.inf)
        ps = ps.masked_fill(~anchor_active.permute(0, 2, 1).unsqueeze(-1), -torch.inf)
        top, pidx = ps.topk(kc, dim=-1)
        pidx, top = pidx.permute(0, 2, 1, 3), top.permute(0, 2, 1, 3)
        pact = torch.isfinite(top)
        partner = self.gather(memory, pidx)
        ao = self.operand(anchor).unsqueeze(3).expand(-1, -1, -1, kc, -1)
        po = self.operand(partner)
        rel = self.relation_mlp(torch.cat((ao, po, ao * po, ao - po), -1))
        pw = top.masked_fill(~pact, -1.0e4).softmax(-1) * pact
        pw = pw / pw.sum(-1, keepdim=True).clamp_min(1.0e-9)
        sc = (pw.unsqueeze(-1) * rel).sum(3) * anchor_active.unsqueeze(-1).to(rel.dtype)
        sw = self.slot_mix_logits.softmax(0)[None, None, :] * anchor_active
        sw = sw / sw.sum(-1, keepdim=True).clamp_min(1.0e-9)
        context = (sc * sw.unsqueeze(-1)).sum(2)
        out = hidden + torch.sigmoid(self.residual_gate) * context
        return out, {"anchor_index": anchor_index, "partner_index": pidx, "top": top,
                     "normalized": x, "context": context}
