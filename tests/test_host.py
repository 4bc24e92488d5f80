"""Host-side request bookkeeping (no GPU): seeding of DecodeControl."""
from zllm_amd.engine import DecodeControl


def test_unseeded_requests_get_distinct_keys():
    # sampler.rs:26-29: no seed -> thread RNG; here a fresh OS-entropy key
    keys = {DecodeControl(seed=None).seed for _ in range(64)}
    assert len(keys) == 64
    assert all(0 <= k < 2**64 for k in keys)
    assert not DecodeControl(seed=None).seeded


def test_seeded_request_keeps_its_seed():
    d = DecodeControl(seed=1234)
    assert d.seed == 1234 and d.seeded
    assert DecodeControl(seed=-1).seed == 2**64 - 1
