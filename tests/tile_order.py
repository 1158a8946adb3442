"""Host emulation of the ring kernels' tile order, for tests."""
import torch


def split_tile_mask(m, n, tw, tt, group_t, tiles_w, tiles_t, first):
    """Boolean (m, n) mask of the tiles with grouped index >= first: the
    grouped tile order of the ring kernels (runs of group_t token tiles sweep
    the weight tiles together; reference kernels/baseline_triton.py:36-45)."""
    mask = torch.zeros(m, n, dtype=torch.bool)
    per_group = group_t * tiles_w
    for tile in range(first, tiles_w * tiles_t):
        first_t = (tile // per_group) * group_t
        gsize = min(tiles_t - first_t, group_t)
        local = tile % per_group
        pt, pw = first_t + local % gsize, local // gsize
        mask[pt * tt:(pt + 1) * tt, pw * tw:(pw + 1) * tw] = True
    return mask
