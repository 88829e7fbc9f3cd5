"""Argument validation of rsllm_hip_matmul_quant_f32 (host form) and
rsllm_hip_matmul_quant_f32_dev, checked case by case against the oracle's
restatement of quant_matmul.rs:57-92 (dtype guard, in_dim % block with the
NotBlockAligned {what, actual, block} detail, then the weights, x and out
lengths) and the row_len > 0 assertion of parallel.rs:44. Validation runs
before any device work, so these run without a GPU: the device form gets
non-null placeholder addresses that are never dereferenced."""
import numpy as np
import pytest

import kats

F16, Q4_0, Q4_K, Q6_K, Q8_0 = 1, kats.Q4_0, kats.Q4_K, kats.Q6_K, kats.Q8_0

# (weights bytes, x len, out len, n_tok, in_dim, out_dim, dtype)
CASES = [
    # dtype guard first, even with everything else wrong (rejects_unsupported_dtype :156-170)
    ((0, 0, 4, 1, 30, 4, F16), "shape"),
    # in_dim alignment before the weights length (rejects_unaligned_in_dim)
    ((0, 0, 4, 1, 30, 4, Q4_0), "aligned"),
    ((0, 0, 4, 1, 300, 4, Q4_K), "aligned"),
    ((0, 0, 4, 1, 100, 4, Q6_K), "aligned"),
    ((0, 0, 4, 1, 40, 4, Q8_0), "aligned"),
    # weights before x before out
    ((10, 31, 3, 1, 32, 4, Q8_0), "weights"),
    ((136, 31, 3, 1, 32, 4, Q8_0), "x"),
    ((136, 32, 3, 1, 32, 4, Q8_0), "out"),
    ((4 * 144, 2 * 256, 7, 2, 256, 4, Q4_K), "out"),
    ((4 * 144, 256, 4, 2, 256, 4, Q4_K), "x"),          # x must be n_tok * in_dim
    ((3 * 144, 256, 4, 1, 256, 4, Q4_K), "weights"),
    # out_dim == 0 passes the length checks and then trips parallel.rs:44
    ((0, 32, 0, 1, 32, 0, Q8_0), "panic"),
]


def _oracle_status(O, case):
    wb, xl, ol, n_tok, in_dim, out_dim, dt = case
    rc, _ = O.matmul_quant_f32(np.zeros(wb, np.uint8), np.zeros(xl, np.float32), n_tok, in_dim,
                               out_dim, dt, allow_q6k=True, out_len=ol)
    return rc, O.last_detail() if rc == O.NOT_BLOCK_ALIGNED else None


def _call_host(hip, case):
    wb, xl, ol, n_tok, in_dim, out_dim, dt = case
    hip.matmul_quant_f32(np.zeros(ol, np.float32), np.zeros(wb, np.uint8),
                         np.zeros(xl, np.float32), n_tok, in_dim, out_dim, dt)


def _call_dev(hip, case):
    wb, xl, ol, n_tok, in_dim, out_dim, dt = case
    fake = 1 << 40  # never dereferenced: every case fails validation
    hip.matmul_quant_f32_dev(fake, ol, fake, wb, fake, xl, n_tok, in_dim, out_dim, dt, 0)


@pytest.mark.parametrize("form", ["host", "dev"])
@pytest.mark.parametrize("case,kind", CASES)
def test_validation_matches_oracle(hip, oracle, form, case, kind):
    O = oracle
    rc, detail = _oracle_status(O, case)
    call = _call_host if form == "host" else _call_dev
    with pytest.raises(hip.Error) as ei:
        call(hip, case)
    e = ei.value
    if kind == "panic":
        assert rc == O.PANIC
        assert isinstance(e, hip.InvalidArgument)
        return
    if kind == "aligned":
        assert rc == O.NOT_BLOCK_ALIGNED
        assert isinstance(e, hip.NotBlockAligned)
        # the detail a caller's to_error builds NotBlockAligned{what, actual, block} from
        assert e.what == "in_dim"
        assert (e.actual, e.block) == detail == (case[4], {Q4_0: 32, Q8_0: 32}.get(case[6], 256))
        return
    assert rc == O.SHAPE_MISMATCH
    assert isinstance(e, hip.ShapeMismatch)
    if kind in ("weights", "x", "out"):
        assert f"{kind} must be" in e.message
    else:
        assert "dtype" in e.message


def test_q6k_passes_the_guard_as_a_superset(hip):
    # The reference's guard rejects Q6_K (quant_matmul.rs:57-64); this backend
    # accepts it, so a Q6_K call with a wrong x length fails on x, not dtype.
    with pytest.raises(hip.ShapeMismatch, match="x must be"):
        _call_host(hip, (4 * 210, 255, 4, 1, 256, 4, Q6_K))
