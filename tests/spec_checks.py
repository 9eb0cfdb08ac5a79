"""Oracle check of attention layer calls sampled from the speculative loop.

Used by tests/test_gpu_spec_loop.py and tests/run_spec_loop.py: the sampled
call's q (after the prologue), output and LSE are compared with the numpy
oracle on the referenced KV blocks of that layer (outputs within 2e-3 abs +
1e-2 rel, natural-log LSE within 1e-4).
"""

from __future__ import annotations

import numpy as np
import torch

import oracle
from helpers import ATOL_LSE, ATOL_O, RTOL_O


def make_checker(results: list):
    """Factory of check callbacks for ``nebulasd_amd.spec_loop.run``; each
    appends one result dict to `results`."""

    def make_check():
        def check(model, layer, q, o, lse, seq_ids, seq_lens):
            torch.cuda.synchronize()
            bt = model.block_table.cpu().numpy()
            ids = sorted({int(bt[s, i]) for s, n in zip(seq_ids, seq_lens)
                          for i in range((n + 15) // 16)})
            remap = np.zeros(model.k_cache.shape[0], dtype=np.int64)
            remap[ids] = np.arange(len(ids))
            sel = torch.tensor(ids, device=q.device)
            kc = model.k_cache[sel, layer].unsqueeze(1).cpu().numpy()
            vc = model.v_cache[sel, layer].unsqueeze(1).cpu().numpy()
            want_o, want_l = oracle.paged_attention(q.cpu().numpy(), kc, vc, remap[bt], seq_ids,
                                                    seq_lens, 0)
            got_o, got_l = o.float().cpu().numpy(), lse.cpu().numpy()
            excess = float(np.max(np.abs(got_o - want_o) - RTOL_O * np.abs(want_o)))
            dlse = float(np.max(np.abs(got_l - want_l)))
            _, counts = np.unique(np.asarray(seq_ids), return_counts=True)
            results.append({"layers": model.mc.num_layers, "layer": layer, "rows": len(seq_ids),
                            "max_q_len": int(counts.max()), "max_seq_len": int(max(seq_lens)),
                            "excess_o": excess, "max_dlse": dlse,
                            "ok": bool(excess <= ATOL_O and dlse <= ATOL_LSE)})
        return check

    return make_check
