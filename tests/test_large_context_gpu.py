"""A decode step past the model's context: 1,100,000 keys of head_dim 512, so
each of the K and V caches holds 2.25 GB and every address past the first
2^31 bytes of them comes from 64-bit row offsets. Gemma-4-E2B stops at 131072
keys (configs[2], tested at full size elsewhere); this case checks that
nothing in the host plan (trim, split count, workspace) or in the streaming
decode and combine kernels wraps at 32 bits. Compared with the CPU oracle
(rust/src/backend_cpu.rs:270-336 restated in oracle/attn_oracle.c) at the
north star's bar (1e-5 max-abs, 1e-6 mean-abs)."""
import numpy as np
import pytest

import g4a
import g4a.synth as synth
import oracle

pytestmark = pytest.mark.gpu

S, DH, HQ = 1_100_000, 512, 8


def test_decode_past_two_gigabytes_of_keys(ctx):
    rng = np.random.default_rng(77)
    # numpy's generator rather than the bench's splitmix64 stream: 1.1 G values in a few seconds
    q = synth.rms_norm_rows(rng.standard_normal((1, HQ, DH), dtype=np.float32))
    k = synth.rms_norm_rows(rng.standard_normal((S, 1, DH), dtype=np.float32))
    v = rng.standard_normal((S, 1, DH), dtype=np.float32)
    assert k.nbytes > 2 ** 31
    plan = ctx.plan(T=1, S=S, Hq=HQ, Hkv=1, Dh=DH, Dv=DH, q_pos0=S - 1, k_pos0=0)
    print(f"[gpu] decode over {S} keys ({k.nbytes / 2**30:.2f} GiB of K): kernel "
          f"{g4a.KERNEL_NAMES[plan.kernel]}, {plan.splits} splits of {plan.keys_per_split} keys", flush=True)
    want = oracle.attention(q, k, v, np.array([S - 1], np.uint32), np.arange(S, dtype=np.uint32))
    got = g4a.attention_host(ctx, q, k, v)
    d = np.abs(got.astype(np.float64) - want.astype(np.float64))
    print(f"  max-abs {d.max():.3e} mean-abs {d.mean():.3e}", flush=True)
    assert d.max() <= 1e-5 and d.mean() <= 1e-6
