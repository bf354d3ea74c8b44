"""GPU parity over a seeded random sweep of shapes.

Each case draws a batch, head layout, head_dim, q_len, cache dtype (e4m3fn, fp16,
bf16; a second range of seeds uses e5m2 caches), scale
kind, ragged lengths (empty sequences and page-boundary lengths included),
split size, workspace dtype and (fp8, q_len > 1) arbitrary tree-mask words
from a fixed seed, runs the op (a third seed range with the single-launch
kernel's split mode forced), and compares
with the CPU oracle at the tolerances in ``pd_helpers``.  Sizes stay small so
that the oracle finishes each case in well under a second.
"""

import numpy as np
import pytest
import torch

import pd_helpers as H

pytestmark = pytest.mark.gpu

N_CASES = 120
N_E5M2 = 24
SPLITS = [64, 96, 128, 256, 512, 1024]
HEADS = [(4, 4), (8, 2), (14, 2), (16, 8), (28, 4), (32, 4)]


@pytest.fixture(scope="module", autouse=True)
def _require_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X GPU")
    import l20_paged_decode  # noqa: F401  (fails loudly if the extension is missing)


def draw(case, seed_base=1000):
    rng = np.random.default_rng(seed_base + case)
    hq, hkv = HEADS[rng.integers(len(HEADS))]
    d = int(rng.choice([64, 128]))
    q_len = int(rng.choice([1, 1, 2, 4]))
    if (hq // hkv) * q_len > 32:
        q_len = 1
    batch = int(rng.integers(1, 9))
    kind = rng.integers(4)
    if kind == 0:  # short and ragged around page boundaries
        lens = rng.choice([0, 1, 15, 16, 17, 31, 32, 33, 63, 64, 65], size=batch)
    elif kind == 1:  # medium
        lens = rng.integers(1, 1500, size=batch)
    elif kind == 2:  # one long, the rest short
        lens = rng.integers(0, 100, size=batch)
        lens[rng.integers(batch)] = rng.integers(2000, 5000)
    else:  # equal lengths
        lens = np.full(batch, int(rng.integers(100, 3000)))
    lens = [max(int(x), q_len if x > 0 else 0) for x in lens]
    return dict(hq=hq, hkv=hkv, d=d, q_len=q_len, batch=batch, lens=lens,
                cache=str(rng.choice(["fp8", "fp8", "fp16", "bf16"])),
                per_head=bool(rng.integers(2)),
                split=int(rng.choice(SPLITS)),
                partial=str(rng.choice(["fp32", "fp32", "fp16"])),
                seed=int(rng.integers(1 << 30)),
                tree=bool(q_len > 1 and rng.integers(2)))


def run_case(c):
    pdt = torch.float16 if c["partial"] == "fp16" else torch.float32
    if c["cache"] in ("fp8", "e5m2"):
        inp = H.make_synthetic(c["batch"], c["hq"], c["hkv"], c["d"], c["lens"], q_len=c["q_len"],
                               per_head=c["per_head"], seed=c["seed"], garbage_tail=True,
                               fp8="e5m2" if c["cache"] == "e5m2" else "e4m3fn")
        if c["tree"]:  # arbitrary ancestor words over the q_len drafts, one row per (sequence, draft)
            w = np.random.default_rng(c["seed"]).integers(0, 2**32, size=(c["batch"], c["q_len"]), dtype=np.int64)
            inp["tree_mask"] = torch.from_numpy(np.where(w >= 2**31, w - 2**32, w).astype(np.int32)).cuda()
        H.compare(*H.run_op(inp, c["split"], partial_dtype=pdt), *H.run_oracle(inp))
    else:
        dtype = torch.float16 if c["cache"] == "fp16" else torch.bfloat16
        inp = H.make_synthetic16(c["batch"], c["hq"], c["hkv"], c["d"], c["lens"], dtype=dtype,
                                 q_len=c["q_len"], seed=c["seed"], garbage_tail=True, csr_pad=1)
        csr = bool(c["seed"] & 1)
        H.compare(*H.run_op16(inp, c["split"], csr=csr, partial_dtype=pdt), *H.run_oracle16(inp, csr=csr))


@pytest.mark.parametrize("case", range(N_CASES))
def test_random_shape(case):
    c = draw(case)
    print(case, c, flush=True)
    run_case(c)


@pytest.mark.parametrize("case", range(N_E5M2))
def test_random_shape_e5m2(case):
    """Another seed range with OCP e5m2 caches (the draws' other fields as above)."""
    c = dict(draw(case, seed_base=5000), cache="e5m2")
    print(case, c, flush=True)
    run_case(c)


N_SPLIT_MODE = 48


@pytest.mark.parametrize("case", range(N_SPLIT_MODE))
def test_random_shape_split_mode(case, monkeypatch):
    """A third seed range with the single-launch kernel's split mode forced
    (L20_PD_FUSED_SPLIT=1) at the splits it accepts (256, 512, 1024 tokens);
    calls with one split slot still run the persistent kernel."""
    monkeypatch.setenv("L20_PD_FUSED_SPLIT", "1")
    c = draw(case, seed_base=9000)
    c["split"] = int(np.random.default_rng(9000 + case).choice([256, 256, 512, 1024]))
    print(case, c, flush=True)
    run_case(c)
