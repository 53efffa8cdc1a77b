"""Committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_fixtures.py from the oracle).

CPU tests: the oracle still reproduces every fixture, and the fixtures agree
with what the arithmetic fixes in closed form (constant rows rotate to 16x the
constant, e_0 rotates to the sign pattern of the 4-point matrix's first
column, non-finite rows give zero codes and an infinite scale, tied router
logits pick the lowest ids with equal probabilities), so a fixture written by
a broken oracle fails here. GPU tests: the C ABI reproduces every fixture bit
for bit.
"""
import numpy as np
import pytest

import oracle
from golden import make_fixtures as fx

BF = oracle.f32_to_bf16
F = oracle.bf16_to_f32


def nibbles(words: np.ndarray) -> np.ndarray:
    w = words.astype(np.uint32)
    return np.stack([(w >> (4 * p)) & 15 for p in range(8)], axis=-1).reshape(w.shape[0], -1)


def first_column_signs(width: int) -> np.ndarray:
    """Signs of column 0 of [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],[-1,1,1,1]]^{(x)4}:
    entry i is -1 for every base-4 digit of i % 256 equal to 3."""
    i = np.arange(width) % 256
    neg = sum(((i >> (2 * d)) & 3) == 3 for d in range(4))
    return np.where(neg % 2 == 1, -1, 1)


# ------------------------------------------------------------------ CPU side

@pytest.mark.parametrize("name", sorted(fx.MAKERS))
def test_oracle_reproduces_fixture(name):
    want = fx.load(name)
    got = fx.MAKERS[name]()
    assert sorted(got) == sorted(want)
    for key in want:
        assert np.array_equal(np.asarray(got[key]).view(np.uint8), want[key].view(np.uint8)), (name, key)


@pytest.mark.parametrize("width", fx.PREPARE_WIDTHS)
def test_prepare_fixture_closed_forms(width):
    z = fx.load("prepare_rows")
    codes, scales = z[f"codes{width}_4"], z[f"scales{width}_4"]
    nib = nibbles(codes)
    # zero row: codes 0, scale RN(1e-30 / 7)
    assert not nib[0].any() and scales[0] == np.float32(1e-30) / np.float32(7)
    # e_0: group 0 rotates to +-1 everywhere, so its codes are +-7 with the signs
    # of column 0; the other groups are zero
    want = np.where(first_column_signs(width) > 0, 7, 9)
    want[256:] = 0
    assert np.array_equal(nib[1], want)
    assert scales[1] == np.float32(0.0625) / np.float32(7)
    # NaN and Inf rows: all codes zero, scale +inf
    for r in (3, 4):
        assert not nib[r].any() and np.isinf(scales[r])
    # constant rows rotate to 16x the constant: -0.5 -> -8 -> code -7, 19 -> 304 -> code 7
    assert (nib[7] == 9).all() and scales[7] == np.float32(0.5) / np.float32(7)
    assert (nib[8] == 7).all() and scales[8] == np.float32(19.0) / np.float32(7)


def test_route_fixture_closed_forms():
    z = fx.load("route_ties")
    for key in ("routes_f32", "routes_bf16"):
        r = z[key]
        # all-equal and +-0 rows: ids 0..7, probabilities bf16(1/8)
        for t in (0, 1):
            assert np.array_equal(r[t, :8], np.arange(8, dtype=np.float32))
            assert (r[t, 8:] == 0.125).all()
        # four exact maxima of 3.0: they come first, in ascending id order
        logits = z["logits_f32"]
        if logits[2].max() == 3.0:
            assert np.array_equal(r[2, :4], [5, 9, 77, 100])
        # duplicated halves: each tied pair is taken lowest id first
        ids = r[7, :8].astype(int)
        for a, b in zip(ids, ids[1:]):
            assert logits[7, a] > logits[7, b] or (logits[7, a] == logits[7, b] and a < b)


def test_group_fixture_brute_force():
    z = fx.load("group_t33")
    routes, groups, order = z["routes"], z["groups"], z["order"]
    for e in range(128):
        slots = [8 * t + r for t in range(33) for r in range(8) if int(routes[t, r]) == e]
        assert groups[e, 0] == len(slots)
        assert np.array_equal(groups[e, 1:1 + len(slots)], np.array(slots, dtype=np.float32))
    for t in range(33):
        ids = routes[t, :8].astype(int)
        assert np.array_equal(order[t].astype(int), np.argsort(ids, kind="stable"))


# ------------------------------------------------------------------ GPU side

def _gpu():
    import torch

    import clef_i4
    return torch, clef_i4


def _bf16_dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


def _u16(t):
    return t.contiguous().view(__import__("torch").int16).cpu().numpy().view(np.uint16)


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("width", fx.PREPARE_WIDTHS)
def test_gpu_prepare_fixture(width, bits):
    torch, clef_i4 = _gpu()
    z = fx.load("prepare_rows")
    p = clef_i4.prepare(_bf16_dev(torch, z[f"x{width}"]), bits=bits)
    codes = p.codes.cpu().numpy().view(np.uint32)[:, : width * bits // 32]
    assert np.array_equal(codes, z[f"codes{width}_{bits}"])
    assert np.array_equal(p.scales.cpu().numpy().view(np.uint32), z[f"scales{width}_{bits}"].view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_gpu_route_fixture(dtype):
    torch, clef_i4 = _gpu()
    z = fx.load("route_ties")
    logits = z[f"logits_{dtype}"]
    dev = _bf16_dev(torch, logits) if dtype == "bf16" else torch.from_numpy(logits).cuda()
    got = clef_i4.omni_route(dev, 8).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), z[f"routes_{dtype}"].view(np.uint32))


@pytest.mark.gpu
def test_gpu_group_fixture():
    torch, clef_i4 = _gpu()
    z = fx.load("group_t33")
    groups, order = clef_i4.omni_group_routes(torch.from_numpy(z["routes"]).cuda())
    assert np.array_equal(groups.cpu().numpy(), z["groups"])
    assert np.array_equal(order.cpu().numpy(), z["order"])
    tasks = clef_i4.omni_expert_tasks(groups).cpu().numpy()
    n = 1 + 2 * int(z["tasks"][0])
    assert np.array_equal(tasks[:n], z["tasks"][:n])


@pytest.mark.gpu
def test_gpu_gemm_fixture():
    torch, clef_i4 = _gpu()
    z = fx.load("gemm_m5")
    x, w, res = fx.inputs("gemm_m5")
    weight = clef_i4.load_quantized_weight(_bf16_dev(torch, w))
    a = clef_i4.prepare(_bf16_dev(torch, x))
    assert np.array_equal(_u16(clef_i4.project_prepared(a, weight)), z["out"])
    assert np.array_equal(_u16(clef_i4.project_prepared(a, weight, residual=_bf16_dev(torch, res))),
                          z["out_residual"])


@pytest.mark.gpu
def test_gpu_moe_fixture():
    torch, clef_i4 = _gpu()
    z = fx.load("moe_t17")
    x, logits, gate, up, down = fx.inputs("moe_t17")
    layer = clef_i4.MoeLayer(clef_i4.load_quantized_weight(_bf16_dev(torch, gate)),
                             clef_i4.load_quantized_weight(_bf16_dev(torch, up)),
                             clef_i4.load_quantized_weight(_bf16_dev(torch, down)))
    routes = torch.empty((x.shape[0], 16), dtype=torch.float32, device="cuda")
    out = layer(_bf16_dev(torch, x), _bf16_dev(torch, logits), routes_out=routes)
    assert np.array_equal(routes.cpu().numpy().view(np.uint32), z["routes"].view(np.uint32))
    assert np.array_equal(_u16(out), z["out"])
