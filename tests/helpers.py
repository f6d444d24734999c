"""Shared test helpers: seeded inputs and oracle <-> product page conversion."""
import numpy as np

from dotcache_amd.types import EncodedPage, PageHeader


def to_product_page(op) -> EncodedPage:
    """An oracle page as the product's EncodedPage (same arrays, same header)."""
    return EncodedPage(
        header=PageHeader.from_dict(op.header.to_dict()),
        payload=op.payload, scales=op.scales, bias=op.bias,
        escape_payload=op.escape_payload, escape_scales=op.escape_scales,
        runtime_page_mean=op.runtime_page_mean, runtime_page_sketch=op.runtime_page_sketch,
        runtime_page_min=op.runtime_page_min, runtime_page_max=op.runtime_page_max,
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


def pool_page_to_oracle(pool, page_id, kind):
    """Download one device page (written by the product) as an oracle page."""
    from oracle import dotcache_oracle as O

    page = pool.download_page(int(page_id), kind=kind)
    return O.OraclePage(header=O.OracleHeader(**page.header.to_dict()), payload=page.payload, scales=page.scales,
                        bias=page.bias, escape_payload=page.escape_payload, escape_scales=page.escape_scales)


def workload_oracle(wl, layer, b, h):
    """Oracle decode of (layer, sequence b, KV head h) of a built workload:
    ``[n_q, head_dim]`` from the pages as they sit in the pools now."""
    from oracle import dotcache_oracle as O

    lt = wl.layers[layer]
    n = int(lt.seq_pages[b])
    kt = lt.k_table[b, h, :n].cpu().numpy()
    vt = lt.v_table[b, h, :n].cpu().numpy()
    kp = [pool_page_to_oracle(wl.k_pool, p, "K") for p in kt]
    vp = [pool_page_to_oracle(wl.v_pool, p, "V") for p in vt]
    q = wl.queries[layer][b, h].float().cpu().numpy() * wl.query_scale
    return O.decode_multi_query_step(q, kp, vp)[2]
