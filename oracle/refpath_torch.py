"""Torch-CPU restatement of the reference's streaming path -- TEST/BASELINE ONLY.

This is the CPU baseline that ``bench.py`` times beside the GPU path (kind
"port"): it follows the reference's own op sequence on torch CPU tensors so that
its cost is representative of the reference running on the host.  It is not
the product and the product never imports it.

Op sequence restated (reference paths):

* advance, post-freeze: ``tgengine/core/temporal_graph.py:123-129`` -> ``_append_overflow``
  ``:351-387``: cat -> ``from*M+arange`` key -> stable argsort -> two
  ``unique_consecutive`` -> keep last B -> ``index_put_`` x3 -> ``scatter_add_``.
* recent with a ring and an empty CSR: ``:223-280`` -> ``_merge_overflow`` ``:307-349``:
  all-pad CSR part, ring row gather, validity, cat, ``sort`` by time, gather x4, last K.
* DataPipeline.prepare grouping: ``tgengine/pipeline/__init__.py:40-113``.
* FixedCosineTimeEncoder: ``tgengine/nn/time_encoding.py:37-63`` (Linear(1,d) + cos) on
  the DyGFormer dt (``tgengine/models/dygformer.py:273-279``).
* co-occurrence: broadcast (ii) counts as in ``temporal_sample.cu:453-511`` and the (B,)
  pair count of ``tgengine/pipeline/__init__.py:206-219``.
"""
from __future__ import annotations

import numpy as np
import torch

PAD = -1


class RefPathCPU:
    def __init__(self, num_nodes: int, d: int, B: int, d_t: int = 100):
        self.N, self.d, self.B = num_nodes, d, B
        self.ids = torch.full((num_nodes, B), PAD, dtype=torch.int32)
        self.times = torch.zeros((num_nodes, B), dtype=torch.float64)
        self.feats = torch.zeros((num_nodes, B, d), dtype=torch.float32)
        self.wp = torch.zeros(num_nodes, dtype=torch.int64)
        w = 1.0 / (10 ** np.linspace(0, 9, d_t, dtype=np.float32))
        self.lin = torch.nn.Linear(1, d_t, bias=True)
        with torch.no_grad():
            self.lin.weight.copy_(torch.from_numpy(w).reshape(d_t, 1))
            self.lin.bias.zero_()
        self.lin.requires_grad_(False)

    # -- kernel (a) --------------------------------------------------------
    def advance(self, src, dst, time, feat):
        frm = torch.cat([src, dst])
        to = torch.cat([dst, src])
        tt = torch.cat([time, time])
        ff = torch.cat([feat, feat])
        n = frm.shape[0]
        B = self.B
        key = frm.long() * (int(tt.max().item()) + 2) + torch.arange(n)
        perm = key.argsort(stable=True)
        s_from, s_to, s_t, s_f = frm[perm], to[perm], tt[perm], ff[perm]
        _, inv, cnts = torch.unique_consecutive(s_from.long(), return_inverse=True,
                                                return_counts=True)
        gs = torch.cat([torch.zeros(1, dtype=torch.int64), cnts.cumsum(0)[:-1]])
        off = torch.arange(n) - gs[inv]
        keep = off >= (cnts[inv] - B)
        s_from, s_to, s_t, s_f = s_from[keep], s_to[keep], s_t[keep], s_f[keep]
        nk = s_from.shape[0]
        _, inv2, cnts2 = torch.unique_consecutive(s_from.long(), return_inverse=True,
                                                  return_counts=True)
        gs2 = torch.cat([torch.zeros(1, dtype=torch.int64), cnts2.cumsum(0)[:-1]])
        koff = torch.arange(nk) - gs2[inv2]
        widx = (self.wp[s_from] + koff) % B
        self.ids[s_from, widx] = s_to.to(torch.int32)
        self.times[s_from, widx] = s_t.to(torch.float64)
        self.feats[s_from, widx] = s_f
        self.wp.scatter_add_(0, s_from.long(), torch.ones(nk, dtype=torch.int64))

    # -- kernel (b) --------------------------------------------------------
    def recent(self, nodes, qt, K):
        Q = nodes.shape[0]
        c_ids = torch.full((Q, K), PAD, dtype=torch.int32)
        c_t = torch.zeros(Q, K, dtype=torch.float64)
        c_f = torch.zeros(Q, K, self.d, dtype=torch.float32)
        c_m = torch.zeros(Q, K, dtype=torch.bool)
        safe = nodes.clamp(min=0)
        r_ids = self.ids[safe]
        r_t = self.times[safe]
        r_f = self.feats[safe]
        r_v = (r_ids != PAD) & (r_t < qt.unsqueeze(1))
        if r_v.sum() == 0:
            return c_ids, c_t, c_f, c_m
        a_ids = torch.cat([c_ids, r_ids], 1)
        a_t = torch.cat([c_t, r_t], 1)
        a_f = torch.cat([c_f, r_f], 1)
        a_m = torch.cat([c_m, r_v], 1)
        _, order = a_t.masked_fill(~a_m, -float("inf")).sort(dim=1)
        a_ids = torch.gather(a_ids, 1, order)
        a_t = torch.gather(a_t, 1, order)
        a_f = torch.gather(a_f, 1, order.unsqueeze(-1).expand(-1, -1, self.d))
        a_m = torch.gather(a_m, 1, order)
        T = a_ids.shape[1]
        return a_ids[:, T - K:], a_t[:, T - K:], a_f[:, T - K:], a_m[:, T - K:]

    # -- prepare = grouping + recent + time-enc (+ co-occurrence) ------------
    def prepare(self, src, dst, neg, time, K, co: bool = False):
        groups = [src, dst, neg.reshape(-1)]
        tl = [time, time,
              time.unsqueeze(1).expand_as(neg).reshape(-1) if neg.ndim > 1 else time]
        nodes = torch.cat(groups)
        qt = torch.cat(tl)
        ids, t, f, m = self.recent(nodes, qt, K)
        dt = qt.unsqueeze(1).float() - t.float()
        te = torch.cos(self.lin(dt.unsqueeze(-1)))
        te = te.masked_fill(~m.unsqueeze(-1), 0.0)
        out = {"ids": ids, "times": t, "feats": f, "mask": m, "te": te}
        if co:
            b = src.shape[0]
            a, c = ids[:b], ids[b:2 * b]
            am, cm = m[:b], m[b:2 * b]
            eq_ac = a.unsqueeze(2) == c.unsqueeze(1)
            a_cnt = torch.stack([(a.unsqueeze(2) == a.unsqueeze(1)).sum(2), eq_ac.sum(2)], -1)
            c_cnt = torch.stack([eq_ac.sum(1), (c.unsqueeze(2) == c.unsqueeze(1)).sum(2)], -1)
            a_cnt = a_cnt.masked_fill((a == PAD).unsqueeze(-1), 0).to(torch.int32)
            c_cnt = c_cnt.masked_fill((c == PAD).unsqueeze(-1), 0).to(torch.int32)
            pair = (eq_ac & (am.unsqueeze(2) & cm.unsqueeze(1))).any(dim=2).float().sum(dim=1)
            out.update(co_a=a_cnt, co_c=c_cnt, co_pair=pair)
        return out
