"""Inputs of the reference's single-head query example
(sglang/srt/layers/attention/v1_deepseek/example_v1_query_single_head.py:11-54),
built on the CPU from the fixture's page permutations: unique non-negative dot
products, one K head, members reversed inside each 1K bucket, 64 built pages of
a 128-page reordered pool.
"""
import json
from pathlib import Path

import torch

B, P, CAP, TAKE, N, TOP, WINDOW, SINK = 1024, 128, 128, 40, 4097, 2048, 64, 64
_EXAMPLE = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())["route_example"]


def route_inputs(rows=B):
    native_pages = torch.tensor(_EXAMPLE["native_pages"], dtype=torch.int32)
    reorder_pages = torch.tensor(_EXAMPLE["reorder_pages"], dtype=torch.int32)
    nt = native_pages[None].expand(rows, -1).contiguous()
    rt = reorder_pages[None].expand(rows, -1).contiguous()
    k = torch.zeros((N, 128))
    k[:, 0] = torch.arange(N) / 8192
    q = torch.zeros((rows, 128))
    q[:, 0] = 1
    logical_order = torch.arange(4096, dtype=torch.int32).view(4, 1024).flip(1).reshape(64, 64)
    members = torch.full((CAP, 64), -1, dtype=torch.int32)
    members[reorder_pages[:64].long()] = logical_order
    centers = k[logical_order.long()].reshape(64, 8, 8, 128).mean(2)
    scores = torch.full((rows, P * 8), float("-inf"))
    scores[:, :512] = q @ centers.reshape(-1, 128).T
    return dict(nt=nt, rt=rt, k=k, q=q, members=members, scores=scores,
                lens=torch.full((rows,), N, dtype=torch.int32), takes=torch.full((rows,), TAKE, dtype=torch.int32),
                tail_rows=torch.zeros(rows, dtype=torch.int32))


def fine_inputs(d, fine_table):
    """Candidate layout after route: the 40 selected pages' members, sink, tail."""
    rows = fine_table.shape[0]
    tail = max(SINK, min((N - 1) // 1024 * 1024, max(SINK, N - WINDOW)))
    chosen = d["members"][fine_table[:, :TAKE].long()].reshape(rows, -1)
    fixed = torch.cat((torch.arange(SINK), torch.arange(tail, N))).to(torch.int32)
    candidate_ids = torch.cat((chosen, fixed[None].expand(rows, -1)), dim=1)
    fine_scores = (d["q"] @ d["k"][candidate_ids[0].long()].T).contiguous()
    valid = torch.ones_like(candidate_ids, dtype=torch.bool)
    valid[:, :TAKE * 64] = (chosen >= SINK) & (chosen < tail)
    reference_scores = fine_scores.masked_fill(~valid, float("-inf"))
    return dict(candidate_ids=candidate_ids, fine_scores=fine_scores, reference_scores=reference_scores,
                fine_lens=torch.full((rows,), fine_scores.shape[1], dtype=torch.int32))
