"""The reference's CPU path of the decode read, restated with torch on host tensors.

TEST INFRASTRUCTURE ONLY: bench.py's CPU-baseline leg times it, tests/ pin it;
product code never imports it.

lookup() is the torch resolver of adaptive_sparse/request_residency.py:819-825
(Top-K blocks -> positions -> validity -> req_to_token -> mapping, invalid
lanes -1), followed by the miss list the HIP path also produces
(torch.nonzero of valid lanes whose slot is 0, row-major, as
docs/MINIMAX_VMM_LAYOUT.md:54-56 defines slot 0 = not resident). gather() is
the gather of experimental/sparse_read.py:11-30 in its multi-plane form:
index_select of each K/V plane's slot rows, zero rows for slots outside
[zero_below, rows). tests/test_oracle.py pins both against the reference's
smoke vectors and the numpy oracle.
"""

import torch


def lookup(topk, req_to_token, mapping, rows, lengths, selected, block_size):
    """Slots [S, K * bs] int32 of the selected rows and their miss list ([n, 2] (row index, lane) pairs).

    topk [B, K] (layer 0 of the reference's [1, B, K]); req_to_token [R, T];
    mapping [N]; rows, lengths [B]; selected [S].
    """
    blocks = topk[selected].long()
    positions = blocks.unsqueeze(-1) * block_size + torch.arange(block_size)
    positions = positions.flatten(1)
    valid = (positions >= 0) & (positions < lengths[selected, None])
    logical = req_to_token[rows[selected, None], positions.masked_fill(~valid, 0)]
    slots = mapping[logical].masked_fill(~valid, -1).to(torch.int32)
    misses = torch.nonzero(valid & (slots == 0))
    return slots, misses


def gather(planes, slots, zero_below=1):
    """Rows of each plane at `slots` ([n] int32): [P, n, row] with zero rows outside [zero_below, rows).

    planes [P, rows, row] - the K and V planes of one layer.
    """
    inside = (slots >= zero_below) & (slots < planes.shape[1])
    index = torch.where(inside, slots, torch.zeros_like(slots)).long()
    rows = torch.stack([plane.index_select(0, index) for plane in planes])
    return rows.masked_fill_(~inside.view(1, -1, 1), 0)
