"""A seeded random sweep of the batched decode entry point
(g4a_attention_decode_batch) through the C-ABI against the CPU oracle
(rust/src/backend_cpu.rs:270-336 restated in oracle/attn_oracle.c), at the
north star's bar (1e-5 max-abs, 1e-6 mean-abs) for every step of a batch.

Across the batches the draws cover contexts from one key to tens of
thousands, sliding windows over linear caches and over rings of any size at
least the window, full attention, one or two kv heads, both head dims and
caches whose keys sit at explicit positions with holes. A batch is one layer's calls (they
share head dim, kv heads, window and ring capacity) and every one of them must
batch; calls of another layer mixed in run as single calls and must still be
right. Batch sizes cross the 64-sequence launch boundary. The draws come from
one seed."""
import numpy as np
import pytest

from test_decode_batch_gpu import KposSeq, Seq

pytestmark = pytest.mark.gpu

MAX_ABS = 1e-5
MEAN_ABS = 1e-6
N_BATCHES = 8


def draw_batch(rng, b):
    """One layer's calls (they share head dim, kv heads, window and ring capacity,
    as a batch must), contiguous or at explicit positions, with a few calls of
    other layers mixed in (those run as single calls)."""
    n = int(rng.choice([1, 5, 17, 63, 64, 65, 80]))
    Dh = int(rng.choice([256, 512]))
    Hkv = int(rng.choice([1, 1, 2]))
    kind = str(rng.choice(["ring", "linear_window", "global", "kpos"]))
    window = int(rng.choice([512, int(rng.integers(1, 600))])) if kind == "ring" else \
        int(rng.integers(1, 2000)) if kind == "linear_window" else \
        int(rng.choice([0, 512, int(rng.integers(1, 3000))])) if kind == "kpos" else 0
    cap = int(rng.choice([window, window + int(rng.integers(0, 200))])) if kind == "ring" else 0
    seqs = []
    for i in range(n):
        if kind == "kpos":
            S = int(rng.integers(2, 5000))
            seqs.append(dict(kind="kpos", S=S, Dh=Dh, window=window, q_at=int(rng.integers(0, S))))
        else:
            top = 40000 if kind == "ring" else 12000 if kind == "linear_window" else 20000
            L = int(rng.choice([int(rng.integers(1, 40)), int(rng.integers(1, top))]))
            seqs.append(dict(kind="seq", L=L, Dh=Dh, window=window, cap=cap, Hkv=Hkv))
    # calls of another layer (after the first call, which sets the batch's layer
    # fields), which the batch leaves to single calls
    for _ in range(int(rng.integers(0, 3))):
        seqs.insert(int(rng.integers(1, len(seqs) + 1)),
                    dict(kind="seq", L=int(rng.integers(1, 3000)), Dh=768 - Dh, window=0, cap=0, Hkv=1,
                         other=True))
    return seqs


BATCHES = [draw_batch(np.random.default_rng(5000 + b), b) for b in range(N_BATCHES)]


@pytest.mark.parametrize("b", range(N_BATCHES), ids=[f"batch{b}" for b in range(N_BATCHES)])
def test_random_decode_batch(ctx, b):
    spec = BATCHES[b]
    rng = np.random.default_rng(5500 + b)
    kinds = {}
    for s in spec:
        kinds[s["kind"]] = kinds.get(s["kind"], 0) + 1
    print(f"[gpu] batch {b}: {len(spec)} calls {kinds}", flush=True)
    seqs = []
    try:
        for i, s in enumerate(spec):
            seed = 10000 * (b + 1) + i
            if s["kind"] == "seq":
                seqs.append(Seq(ctx, s["L"], s["Dh"], seed=seed, window=s["window"], cap=s["cap"], Hkv=s["Hkv"]))
            else:
                seqs.append(KposSeq(ctx, s["S"], s["Dh"], seed, s["window"], s["q_at"], rng))
        n = ctx.attention_decode_batch([x.kw() for x in seqs])
        print(f"  {n} of {len(seqs)} calls batched", flush=True)
        assert n == sum(1 for s in spec if not s.get("other")), f"batch {b}: {n} calls batched"
        worst_mx, worst_mean = 0.0, 0.0
        for i, (x, s) in enumerate(zip(seqs, spec)):
            d = np.abs(x.out.to_host().astype(np.float64) - x.want().astype(np.float64))
            mx, mean = float(d.max()), float(d.mean())
            worst_mx, worst_mean = max(worst_mx, mx), max(worst_mean, mean)
            assert mx <= MAX_ABS and mean <= MEAN_ABS, f"batch {b} call {i} {s}: max-abs {mx:.3e} mean-abs {mean:.3e}"
        print(f"  worst max-abs {worst_mx:.3e}, worst mean-abs {worst_mean:.3e}", flush=True)
    finally:
        for x in seqs:
            x.free()
