"""Shared test helpers: seeded inputs and oracle <-> product page conversion."""
import numpy as np

from dotcache_amd.types import EncodedPage, PageHeader


def to_product_page(op) -> EncodedPage:
    """An oracle page as the product's EncodedPage (same arrays, same header)."""
    return EncodedPage(
        header=PageHeader.from_dict(op.header.to_dict()),
        payload=op.payload, scales=op.scales, bias=op.bias,
        escape_payload=op.escape_payload, escape_scales=op.escape_scales,
    )


def hard_values(rng, t, hd, *, outliers=True):
    """Normal values plus the cases that stress an encoder: outlier channels,
    constant groups, exact ties on a half-step grid, signed zeros."""
    x = rng.normal(size=(t, hd)).astype(np.float32)
    if outliers and hd >= 8:
        x[:, [1, hd // 3, hd // 2 + 1, hd - 2]] *= 16.0
    if t > 2:
        x[1, : min(hd, 32)] = 2.5           # constant group
        x[2, :] = np.round(x[2, :] * 2) / 2  # half-step grid (ties)
    if t > 3:
        x[3, 0] = -0.0
    return x
