"""zs_spec_verify_static (the entry point that allocates nothing) against
zs_spec_verify on the same inputs: identical accepted counts and tokens, on
two calls in a row, the second with a smaller batch, in both the greedy and
the rejection-sampling mode."""
import ctypes as C

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(B, V, k, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    peak = torch.randint(0, V, (B, k + 1), device="cuda", generator=g)
    tgt = torch.randn((B, k + 1, V), device="cuda", generator=g) * 2.0
    tgt.scatter_add_(2, peak[:, :, None], torch.full((B, k + 1, 1), 12.0, device="cuda"))
    dft = (tgt[:, :k, :] + torch.randn((B, k, V), device="cuda", generator=g) * 0.5).contiguous()
    ids = peak[:, :k].to(torch.int32).contiguous()
    temp = torch.linspace(0.0, 1.2, B, device="cuda")   # row 0 greedy, the rest sampled
    sd = torch.arange(B, dtype=torch.int64, device="cuda") + 11 * seed
    ctr = torch.full((B,), seed, dtype=torch.int64, device="cuda")
    return tgt, dft, ids, temp, sd, ctr


def _static(tgt, dft, ids, temp, sd, ctr):
    from zllm_amd._lib import SpecBatch, lib
    B, kp1, V = tgt.shape
    acc = torch.full((B,), -1, dtype=torch.int32, device="cuda")
    nxt = torch.full((B,), -1, dtype=torch.int32, device="cuda")
    sb = SpecBatch()
    sb.B, sb.V, sb.k, sb.ld = B, V, kp1 - 1, tgt.stride(1)
    sb.d_target, sb.d_draft, sb.d_draft_ids = tgt.data_ptr(), dft.data_ptr(), ids.data_ptr()
    sb.d_temperature, sb.d_seed, sb.d_counter = temp.data_ptr(), sd.data_ptr(), ctr.data_ptr()
    sb.d_accepted, sb.d_next = acc.data_ptr(), nxt.data_ptr()
    sb.flags = 0
    rc = lib().zs_spec_verify_static(C.byref(sb), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, rc
    return acc, nxt


@pytest.mark.parametrize("with_draft", [True, False])
def test_static_matches_context_entry_point(with_draft):
    from tests.gpu_util import ctx
    from zllm_amd.engine import verify_drafts
    c = ctx()
    for B, V, k, seed in ((48, 151936, 4, 1), (9, 32000, 3, 2)):   # second call: smaller input
        print(f"[case] static spec verify B={B} V={V} k={k} draft={with_draft}", flush=True)
        tgt, dft, ids, temp, sd, ctr = _inputs(B, V, k, seed)
        d = dft if with_draft else None
        a_ref, n_ref = verify_drafts(c, tgt, ids, temp, sd, ctr, d)
        if with_draft:
            a_st, n_st = _static(tgt, dft, ids, temp, sd, ctr)
        else:
            a_st, n_st = _static_nodraft(tgt, ids, temp, sd, ctr)
        torch.cuda.synchronize()
        assert torch.equal(a_ref, a_st) and torch.equal(n_ref, n_st)


def _static_nodraft(tgt, ids, temp, sd, ctr):
    from zllm_amd._lib import SpecBatch, lib
    B, kp1, V = tgt.shape
    acc = torch.full((B,), -1, dtype=torch.int32, device="cuda")
    nxt = torch.full((B,), -1, dtype=torch.int32, device="cuda")
    sb = SpecBatch()
    sb.B, sb.V, sb.k, sb.ld = B, V, kp1 - 1, tgt.stride(1)
    sb.d_target, sb.d_draft, sb.d_draft_ids = tgt.data_ptr(), None, ids.data_ptr()
    sb.d_temperature, sb.d_seed, sb.d_counter = temp.data_ptr(), sd.data_ptr(), ctr.data_ptr()
    sb.d_accepted, sb.d_next = acc.data_ptr(), nxt.data_ptr()
    rc = lib().zs_spec_verify_static(C.byref(sb), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, rc
    return acc, nxt


def test_static_rejects_oversize_batch():
    from zllm_amd._lib import SpecBatch, ZS_ELIMIT, lib
    sb = SpecBatch()
    sb.B, sb.V, sb.k, sb.ld = 4097, 8, 1, 8
    sb.d_target = sb.d_draft_ids = sb.d_temperature = sb.d_seed = sb.d_counter = 256
    sb.d_accepted = sb.d_next = 256
    assert lib().zs_spec_verify_static(C.byref(sb), None) == ZS_ELIMIT
    sb.B, sb.V, sb.k, sb.ld = 2000, 151936, 4, 151936    # 2000 * 9 * 19 records > 65536
    sb.d_draft = 256
    assert lib().zs_spec_verify_static(C.byref(sb), None) == ZS_ELIMIT
