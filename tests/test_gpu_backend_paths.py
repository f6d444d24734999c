"""Backend entry points beyond single-query decode, against the oracle:
``decode_multi_query_step`` with more queries than one score pass holds, the
batched grouped decode that returns logits and weights (and its agreement
with the fused output-only path), and the ExecutionTrace byte counters."""
import numpy as np
import pytest

from oracle import dotcache_oracle as O
from tests.helpers import hard_values, to_product_page

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def fresh_pools():
    from dotcache_amd.backends import clear_prepared_pools
    from dotcache_amd.decode import set_decode_path

    clear_prepared_pools()
    set_decode_path("auto")
    yield
    clear_prepared_pools()


def _pages(x, tpp, hd, kind, **fmt):
    return O.encode_pages(x, tokens_per_page=tpp, head_dim=hd, group_size=32, kind=kind, **fmt)


@pytest.mark.parametrize("Q", [7, 12])
def test_decode_multi_query_step_matches_oracle(Q):
    """Q = 12 needs the score kernel's second pass of 8 queries (grid.y = 2)."""
    from dotcache_amd import attention_runtime as rt

    rng = np.random.default_rng(1200 + Q)
    hd = 128
    kp = _pages(hard_values(rng, 150, hd), 64, hd, "K", bits=4)
    vp = _pages(hard_values(rng, 150, hd), 64, hd, "V", bits=4, scheme="symmetric")
    q = (rng.normal(size=(Q, hd)) / np.sqrt(hd)).astype(np.float32)
    logits, weights, out = rt.decode_multi_query_step(q, [to_product_page(p) for p in kp],
                                                      [to_product_page(p) for p in vp], backend="hip_mi355x")
    assert logits.shape == (Q, 150) and weights.shape == (Q, 150) and out.shape == (Q, hd)
    for j in range(Q):
        wl, ww, wo = O.decode_step(q[j], kp, vp)
        np.testing.assert_allclose(logits[j], wl, atol=1e-4, rtol=1e-4, err_msg=f"query {j} logits")
        np.testing.assert_allclose(weights[j], ww, atol=1e-5, rtol=1e-5, err_msg=f"query {j} weights")
        np.testing.assert_allclose(out[j], wo, atol=1e-4, rtol=1e-4, err_msg=f"query {j} output")
    np.testing.assert_allclose(out, O.decode_multi_query_step(q, kp, vp)[2], atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("Q", [2, 12])
def test_grouped_decode_with_logits_matches_oracle_and_output_only(Q):
    """Reference tests/test_torch_cuda_backend.py:505-533: the output-only
    fused path agrees with the full grouped decode (the reference allows
    3e-3; both paths here are within 1e-4 / 3e-4 of the oracle)."""
    import torch

    from dotcache_amd.backends import (decode_grouped_multiquery_step_prepared_hip_tensor,
                                       decode_grouped_multiquery_step_prepared_hip_tensor_output_only,
                                       prepare_pages_hip)

    rng = np.random.default_rng(1300 + Q)
    hd, G, T = 64, 3, 150
    kpg, vpg, qs = [], [], []
    for g in range(G):
        kpg.append(_pages(hard_values(rng, T, hd), 64, hd, "K", bits=4))
        vpg.append(_pages(hard_values(rng, T, hd), 64, hd, "V", bits=4))
        qs.append((rng.normal(size=(Q, hd)) / np.sqrt(hd)).astype(np.float32))
    kprep = [prepare_pages_hip([to_product_page(p) for p in grp]) for grp in kpg]
    vprep = [prepare_pages_hip([to_product_page(p) for p in grp]) for grp in vpg]
    qt = [torch.from_numpy(x).cuda() for x in qs]
    logits, weights, out = decode_grouped_multiquery_step_prepared_hip_tensor(qt, kprep, vprep)
    assert tuple(logits.shape) == (G, Q, T) and tuple(out.shape) == (G, Q, hd)
    logits, weights, out = logits.cpu().numpy(), weights.cpu().numpy(), out.cpu().numpy()
    for g in range(G):
        for j in range(Q):
            wl, ww, wo = O.decode_step(qs[g][j], kpg[g], vpg[g])
            np.testing.assert_allclose(logits[g, j], wl, atol=1e-4, rtol=1e-4, err_msg=f"group {g} query {j}")
            np.testing.assert_allclose(weights[g, j], ww, atol=1e-5, rtol=1e-5, err_msg=f"group {g} query {j}")
            np.testing.assert_allclose(out[g, j], wo, atol=1e-4, rtol=1e-4, err_msg=f"group {g} query {j}")
    fused = decode_grouped_multiquery_step_prepared_hip_tensor_output_only(qt, kprep, vprep).cpu().numpy()
    np.testing.assert_allclose(fused, out, atol=3e-4, rtol=0)
    np.testing.assert_allclose(fused, out, atol=3e-3, rtol=3e-3)  # the reference's own bound


def test_grouped_decode_with_logits_rejects_unequal_groups():
    from dotcache_amd.backends import decode_grouped_multiquery_step_prepared_hip_tensor

    rng = np.random.default_rng(1400)
    kpg = [_pages(hard_values(rng, n, 64), 64, 64, "K", bits=4) for n in (100, 130)]
    vpg = [_pages(hard_values(rng, n, 64), 64, 64, "V", bits=4) for n in (100, 130)]
    qs = [rng.normal(size=(2, 64)).astype(np.float32) for _ in range(2)]
    with pytest.raises(ValueError):
        decode_grouped_multiquery_step_prepared_hip_tensor(qs, [[to_product_page(p) for p in g] for g in kpg],
                                                           [[to_product_page(p) for p in g] for g in vpg])


def test_execution_trace_counts_page_bytes():
    """record_page_read of reference tracing.py:69-71 per page read (payload
    and metadata bytes by the reference's convention), device bytes = the
    compressed bytes of the valid tokens, host-to-device bytes on
    preparation."""
    from dotcache_amd import attention_runtime as rt
    from dotcache_amd.tracing import ExecutionTrace

    rng = np.random.default_rng(1500)
    hd = 128
    kp = _pages(hard_values(rng, 150, hd), 64, hd, "K", bits=4)
    vp = _pages(hard_values(rng, 150, hd), 64, hd, "V", mode="M3")
    kpp, vpp = [to_product_page(p) for p in kp], [to_product_page(p) for p in vp]
    q = rng.normal(size=(3, hd)).astype(np.float32)
    tr = ExecutionTrace()
    rt.decode_multi_query_step(q, kpp, vpp, backend="hip_mi355x", trace=tr)
    pages = kpp + vpp
    assert tr.payload_bytes_read == sum(p.payload_nbytes for p in pages)
    assert tr.metadata_bytes_read == sum(p.metadata_nbytes for p in pages)
    assert tr.device_bytes_read == sum(O.page_device_nbytes(p) for p in kp + vp)
    # by hand: M0 affine 4-bit hd 128 = 4 groups x 4 words x 4 B of codes + 2 x 4 x 2 B of
    # scale and bias per token; M3 fp16 = 256 B per token
    assert tr.device_bytes_read == 150 * (64 + 16) + 150 * 256
    assert tr.host_to_device_bytes == tr.device_bytes_read  # every page prepared once, here
    assert tr.calls["decode_multi_query_step"] == 1
    tr2 = ExecutionTrace()
    rt.score_page(q[0], kpp[2], backend="hip_mi355x", trace=tr2)  # the partial page: 22 tokens
    assert tr2.device_bytes_read == 22 * 80 and tr2.payload_bytes_read == kpp[2].payload_nbytes


def test_cached_page_logits_are_used_and_their_pages_not_read():
    """decode_step_with_page_logits with a mix of cached and None entries
    (reference attention_runtime.py:298-303): the cached logits differ from a
    rescore of their pages, so the output shows they were used, and the trace
    counts only the key pages actually scored, plus every value page."""
    from dotcache_amd import attention_runtime as rt
    from dotcache_amd.tracing import ExecutionTrace

    rng = np.random.default_rng(1600)
    hd = 128
    n = 64 * 4 + 30
    kp = _pages(hard_values(rng, n, hd), 64, hd, "K", bits=4)
    vp = _pages(hard_values(rng, n, hd), 64, hd, "V", bits=4, scheme="symmetric")
    kpp, vpp = [to_product_page(p) for p in kp], [to_product_page(p) for p in vp]
    q = (rng.normal(size=hd) / np.sqrt(hd)).astype(np.float32)
    # pages 1 and 4 (the partial one) cached, perturbed away from their true logits
    cached = [None] * len(kp)
    for i in (1, 4):
        cached[i] = (O.score_page_ref(q, kp[i]) + rng.normal(scale=2.0, size=kp[i].header.token_count)).astype(np.float32)
    tr = ExecutionTrace()
    logits, weights, out = rt.decode_step_with_page_logits(q, kpp, vpp, page_logits=cached, backend="hip_mi355x",
                                                           trace=tr)
    wl, ww, wo = O.decode_step(q, kp, vp, page_logits=cached)
    np.testing.assert_allclose(logits, wl, atol=1e-4, rtol=1e-4)
    np.testing.assert_allclose(weights, ww, atol=1e-6, rtol=1e-4)
    assert np.max(np.abs(out - wo)) < 1e-3
    # a rescore would give a different output
    _, _, fresh = O.decode_step(q, kp, vp)
    assert np.max(np.abs(fresh - wo)) > 1e-2
    scored = [p for i, p in enumerate(kpp) if cached[i] is None]
    assert tr.payload_bytes_read == sum(p.payload_nbytes for p in scored + vpp)
    assert tr.device_bytes_read == sum(O.page_device_nbytes(p) for i, p in enumerate(kp) if cached[i] is None) + \
        sum(O.page_device_nbytes(p) for p in vp)
    # every page cached: no key page is read, the output still follows the cache
    all_cached = [O.score_page_ref(q, p) + 0.5 * rng.normal(size=p.header.token_count).astype(np.float32) for p in kp]
    tr2 = ExecutionTrace()
    _, _, out2 = rt.decode_step_with_page_logits(q, kpp, vpp, page_logits=all_cached, backend="hip_mi355x", trace=tr2)
    assert np.max(np.abs(out2 - O.decode_step(q, kp, vp, page_logits=all_cached)[2])) < 1e-3
    assert tr2.payload_bytes_read == sum(p.payload_nbytes for p in vpp)
