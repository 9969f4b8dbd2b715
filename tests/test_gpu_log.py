"""The log callback on a device: context creation (INFO) and the plans a
call settles on (DEBUG), filtered by the level given with the callback."""
import pytest

import vva
from gpu_util import fill_cache

pytestmark = pytest.mark.gpu


def _decode(torch, c, kv, Hq, d):
    q = torch.randn(kv.n_seq, 1, Hq, d, device="cuda", dtype=torch.float32)
    out = torch.empty_like(q)
    c.attn(kv, 0, q, out, scale=d ** -0.5)
    c.synchronize()


def test_log_callback_reports_context_and_plans(torch_gpu):
    torch = torch_gpu
    got = []
    Hq, Hkv, d, L = 28, 4, 128, 4096
    vva.set_log_callback(lambda lvl, msg: got.append((lvl, msg)), vva.LOG_DEBUG)
    try:
        c = vva.Context(0)
        kv = vva.KVCache(c, 1, Hkv, d, L + 8, 2, vva.Q8_0)
        fill_cache(kv, [L, L], seed=3)
        _decode(torch, c, kv, Hq, d)
        n_debug = sum(1 for lvl, _ in got if lvl == vva.LOG_DEBUG)
        _decode(torch, c, kv, Hq, d)                 # the same plan again: not logged again
        assert sum(1 for lvl, _ in got if lvl == vva.LOG_DEBUG) == n_debug
        kv.free()
        c.close()
        # INFO and above: a new context logs, its plans do not
        vva.set_log_callback(lambda lvl, msg: got.append((lvl, msg)), vva.LOG_INFO)
        c2 = vva.Context(0)
        n0 = len(got)
        kv2 = vva.KVCache(c2, 1, Hkv, d, L + 8, 2, vva.Q8_0)
        fill_cache(kv2, [L, L], seed=4)
        _decode(torch, c2, kv2, Hq, d)
        assert len(got) == n0
        kv2.free()
        c2.close()
    finally:
        vva.set_log_callback(None)
    infos = [m for lvl, m in got if lvl == vva.LOG_INFO]
    debugs = [m for lvl, m in got if lvl == vva.LOG_DEBUG]
    assert len(infos) == 2 and all("device 0" in m and "gfx950" in m for m in infos), infos
    assert n_debug == 1 and "key splits" in debugs[0], debugs
    assert not [m for lvl, m in got if lvl == vva.LOG_ERROR], got
