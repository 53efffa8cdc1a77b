"""Writes the small golden fixtures of this directory from the CPU oracle.

The reference holds no committed INT4 vectors (its tests compute expected
values in-test from formulas and CPU oracles, src/quantized.rs:1068-1150,
src/omni.rs:946-1051), so these fixtures freeze the oracle's outputs on the
reference tests' own input formulas and on seeded inputs. Inputs that are
cheap to regenerate (seeded weights) are rebuilt by `inputs()` below; the
expected outputs are stored.

    python tests/golden/make_fixtures.py      # rewrites *.npz here
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import oracle  # noqa: E402

BF = oracle.f32_to_bf16
F = oracle.bf16_to_f32

PREPARE_WIDTHS = (256, 768, 2048)
MOE = dict(tokens=17, hidden=256, inter=256, seed=1717)
GEMM = dict(m=5, n=256, k=512, seed=505)


def prepare_rows(width: int) -> np.ndarray:
    """bf16 rows: zero, e_0, the formula row ((i*37 % 257) - 128) / 91 of
    rotated_packing_cpu_oracle (src/quantized.rs:1078-1084), and the
    exceptional rows of src/quantized.rs:1138-1150 (NaN at column 259, Inf at
    515, bf16::MAX, a bf16 denormal, -0.5 and 19.0 fills)."""
    base = np.array([((i * 37 % 257) - 128) / 91.0 for i in range(width)], dtype=np.float32)
    rows = [np.zeros(width, np.float32), np.eye(1, width, 0, dtype=np.float32)[0], base]
    for col, bits in ((259, None), (515, None), (3, 0x7F7F), (7, 0x0001)):
        r = F(BF(base)).copy()
        if bits is None:
            r[col % width] = np.nan if col == 259 else np.inf
        else:
            r[col] = F(np.array([bits], dtype=np.uint16))[0]
        rows.append(r)
    rows.append(np.full(width, -0.5, np.float32))
    rows.append(np.full(width, 19.0, np.float32))
    return BF(np.stack(rows))


def route_logits() -> np.ndarray:
    """8 tokens x 128 experts with exact ties, +-0, duplicates of the maximum
    and large magnitudes (the phases of src/benchmarking/omni.rs:43-55)."""
    rng = np.random.default_rng(88)
    x = rng.standard_normal((8, 128)).astype(np.float32)
    x[0, :] = 0.0
    x[1, ::2] = -0.0
    x[1, 1::2] = 0.0
    x[2, [5, 9, 77, 100]] = 3.0
    x[3, :] = np.float32(1e30) * np.sign(x[3])
    x[4, 120:] = 7.5
    x[5, [0, 127]] = 2.0
    x[6] = np.round(x[6] * 2) / 2
    x[7, :64] = x[7, 64:]
    return x


def inputs(name: str):
    """Regenerates the seeded inputs of the fixture `name`."""
    if name == "moe_t17":
        rng = np.random.default_rng(MOE["seed"])
        t, d, i = MOE["tokens"], MOE["hidden"], MOE["inter"]
        x = BF((rng.standard_normal((t, d))).astype(np.float32))
        logits = BF(rng.standard_normal((t, 128)).astype(np.float32))
        gate = BF((rng.standard_normal((128 * i, d)) * 0.02).astype(np.float32))
        up = BF((rng.standard_normal((128 * i, d)) * 0.02).astype(np.float32))
        down = BF((rng.standard_normal((128 * d, i)) * 0.02).astype(np.float32))
        return x, logits, gate, up, down
    if name == "gemm_m5":
        rng = np.random.default_rng(GEMM["seed"])
        m, n, k = GEMM["m"], GEMM["n"], GEMM["k"]
        x = BF(rng.standard_normal((m, k)).astype(np.float32))
        w = BF((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        res = BF(rng.standard_normal((m, n)).astype(np.float32))
        return x, w, res
    raise KeyError(name)


def make_prepare():
    out = {}
    for width in PREPARE_WIDTHS:
        x = prepare_rows(width)
        out[f"x{width}"] = x
        for bits in (4, 8):
            stride = oracle.activation_stride(width, bits)
            codes, scales, _ = oracle.prepare(x, stride, bits)
            out[f"codes{width}_{bits}"] = codes[:, : width * bits // 32]
            out[f"scales{width}_{bits}"] = scales
    return out


def make_route():
    x = route_logits()
    return {"logits_f32": x, "routes_f32": oracle.route(x, 8),
            "logits_bf16": BF(x), "routes_bf16": oracle.route(BF(x), 8)}


def make_group():
    rng = np.random.default_rng(33)
    ids = np.stack([rng.choice(16, 8, replace=False) for _ in range(33)]).astype(np.float32)
    probs = rng.random((33, 8)).astype(np.float32)
    routes = np.concatenate([ids, probs], axis=1)
    groups, order = oracle.group_routes(routes)
    return {"routes": routes, "groups": groups, "order": order, "tasks": oracle.expert_tasks(groups)}


def make_gemm():
    x, w, res = inputs("gemm_m5")
    k, n = GEMM["k"], GEMM["n"]
    stride = oracle.activation_stride(k)
    codes, scales, _ = oracle.prepare(x, stride)
    w_tiled, w_scales = oracle.pack_weight(w)
    return {"out": oracle.gemm(codes, scales, w_tiled, w_scales, n, k),
            "out_residual": oracle.gemm(codes, scales, w_tiled, w_scales, n, k, residual=res)}


def make_moe():
    x, logits, gate, up, down = inputs("moe_t17")
    out, routes = oracle.moe_layer(x, logits, oracle.pack_weight(gate), oracle.pack_weight(up),
                                   oracle.pack_weight(down))
    return {"out": out, "routes": routes}


MAKERS = {"prepare_rows": make_prepare, "route_ties": make_route, "group_t33": make_group,
          "gemm_m5": make_gemm, "moe_t17": make_moe}


def load(name: str):
    with np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


if __name__ == "__main__":
    for name, make in MAKERS.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **make())
        print(path, os.path.getsize(path))
