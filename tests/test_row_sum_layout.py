"""The head_dim 64 prefill takes the softmax's row sums on the matrix cores: P^T's fragment for a
16-key step (the B operand of v_mfma_f32_32x32x16, lane l holding 8 keys of row l % 32) is also
the B operand of one v_mfma_f32_16x16x32 whose A operand is a per-lane 0/1 selector. This checks,
on the CPU, that the selector the kernel builds (csrc/prefill_pp.hip, `sel_word`) gives every lane
the sum of its own row over both halves of the step, under the operand layouts csrc/gfx950.hpp
states for the two instructions. The instructions' layouts themselves are pinned on the GPU by the
head_dim 64 prefill parity tests, which depend on every row sum."""

import numpy as np
import pytest


def kernel_selector(lane):
    # prefill_pp.hip: ((lane >> 4) & 1) == ((lane >> 2) & 1) ? 1.0 : 0.0, the same in all 8 elements.
    return 1.0 if ((lane >> 4) & 1) == ((lane >> 2) & 1) else 0.0


def lane_sums(selector, p):
    """Emulates v_mfma_f32_16x16x32(A = selector per lane, B = the 32x32x16 P^T fragment of p) and
    returns the D registers as [lane][register]."""
    # 32x32x16 B operand: B[k][n] in lane n + 32 (k / 8), element k % 8: lane l holds row l % 32,
    # keys 8 (l / 32) .. + 7 of the step.
    lane_vals = np.array([[p[l % 32, 8 * (l // 32) + e] for e in range(8)] for l in range(64)])
    # 16x16x32 operands: A[m][k] in lane m + 16 (k / 8), element k % 8; B[k][n] likewise with n.
    a = np.array([[selector(m + 16 * (k // 8)) for k in range(32)] for m in range(16)])
    b = np.array([[lane_vals[n + 16 * (k // 8), k % 8] for n in range(16)] for k in range(32)])
    d = a @ b
    # D[m][n] in lane n + 16 (m / 4), register m % 4.
    out = np.zeros((64, 4))
    for m in range(16):
        for n in range(16):
            out[n + 16 * (m // 4), m % 4] = d[m, n]
    return out


def test_every_lane_gets_its_rows_sum():
    rng = np.random.default_rng(0)
    p = rng.random((32, 16))  # P[row][key] of one 16-key step
    got = lane_sums(kernel_selector, p)
    want = np.repeat(p.sum(axis=1)[np.arange(64) % 32][:, None], 4, axis=1)
    np.testing.assert_allclose(got, want, rtol=1e-12)


@pytest.mark.parametrize(
    "wrong",
    [
        lambda l: 1.0,  # all ones: adds rows n and n + 16
        lambda l: 1.0 if ((l >> 4) & 1) == ((l >> 3) & 1) else 0.0,  # wrong output-row bit
        lambda l: 1.0 if ((l >> 5) & 1) == ((l >> 2) & 1) else 0.0,  # wrong key-half bit
        lambda l: 1.0 if ((l >> 4) & 1) != ((l >> 2) & 1) else 0.0,  # the other row's sum
    ],
    ids=["all-ones", "row-bit", "half-bit", "inverted"],
)
def test_a_wrong_selector_is_caught(wrong):
    rng = np.random.default_rng(1)
    p = rng.random((32, 16))
    want = np.repeat(p.sum(axis=1)[np.arange(64) % 32][:, None], 4, axis=1)
    assert not np.allclose(lane_sums(wrong, p), want)
