"""Write the golden fixtures under tests/golden/ from the CPU oracle.

``python tests/golden/make_golden.py`` regenerates them. The fixtures are regression
pins of the oracle itself (its closed-form pins live in tests/test_oracle_*.py):

* ``toy_moe_config1.npz``: BASELINE config 1 (hidden 1024, 8 experts top-2 softmax,
  SwiGLU 512, bf16 weights ~N(0, 0.02), 4 rows ~N(0, 1), torch.manual_seed(0)): the
  inputs' checksums, the routing and the f32 MoE output.
* ``topk_ties.npz``: score vectors with exact ties, +-0 and a count below k, with their
  exact top-k positions by brute force.
"""

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))


def toy_moe_fixture():
    from oracle import moe
    from sgl_amd_mono_amd import workloads

    t = workloads.toy_moe(seed=0)
    ids, w, y = moe.toy_moe(t["x"], t["w_router"], t["w_gate"], t["w_up"], t["w_down"], top_k=2)
    sums = np.array([float(t[k].double().sum()) for k in ("x", "w_router", "w_gate", "w_up", "w_down")])
    np.savez_compressed(HERE / "toy_moe_config1.npz", input_sums=sums, ids=ids.numpy(), weights=w.numpy(),
                        y=y.numpy())


def topk_fixture():
    rng = np.random.default_rng(1234)
    cases = []
    for n, k, levels in ((40, 8, 3), (100, 16, 100), (12, 16, 2), (64, 64, 4), (300, 32, 1)):
        pool = rng.standard_normal(levels).astype(np.float32)
        pool[0] = 0.0
        vals = pool[rng.integers(0, levels, n)]
        if n > 3:
            vals[3] = np.float32(-0.0)
        order = sorted(range(n), key=lambda i: (-float(vals[i]), -np.copysign(1.0, vals[i]), i))
        cases.append((vals, k, np.array(sorted(order[:k]) if n > k else list(range(n)))))
    np.savez_compressed(
        HERE / "topk_ties.npz",
        **{f"vals{i}": c[0] for i, c in enumerate(cases)},
        **{f"k{i}": np.array(c[1]) for i, c in enumerate(cases)},
        **{f"want{i}": c[2] for i, c in enumerate(cases)},
    )


if __name__ == "__main__":
    toy_moe_fixture()
    topk_fixture()
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))
