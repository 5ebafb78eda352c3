"""Host-side layout rules of velograd_amd.kernels.fused_rope_forward against the reference
semantics restated in the oracle (python/velograd/kernels/fused.py:83-129), property-based.

For random q/k shapes and head_dims: where the reference raises, the device API's layout check
raises too; where the reference computes, the device API accepts the inputs, its [outer, seq,
heads, dim] reading of each tensor covers exactly the tensor's elements, and applying the
oracle through that reading reproduces the reference's result.  Four kinds of input the reference
takes through NumPy broadcasting are rejected on purpose (the API requires k's positions to be
q's): a sequence axis of length 1 on one side only (the reference would broadcast one position's
table, or one k row, over the other side), and a k with other leading axes than q (the reference
returns k_rot with q's leading axes); and a head_dim longer than the last axis (the reference
broadcasts the truncated second half and returns a result of another shape than q's); and an odd
head_dim (the reference pairs j with j + head_dim // 2 and drops or broadcasts the unpaired
element)."""

import numpy as np
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle import fused_rmsnorm as ora
from velograd_amd.kernels import _rope_k_layout, _rope_q_layout


def _reference(q_shape, k_shape, head_dim):
    rng = np.random.default_rng(0)
    q = rng.standard_normal(q_shape).astype(np.float32)
    k = rng.standard_normal(k_shape).astype(np.float32) if k_shape is not None else None
    try:
        with np.errstate(all="ignore"):
            return q, k, ora.fused_rope_forward(q, k, head_dim=head_dim)
    except (ValueError, IndexError):
        return q, k, None


def _ours(q_shape, k_shape, head_dim):
    try:
        h_dim = head_dim or q_shape[-1]
        ql, split = _rope_q_layout(tuple(q_shape), h_dim)
        kl = (_rope_k_layout(tuple(k_shape), tuple(q_shape), ql, split, h_dim)
              if k_shape is not None else None)
        return h_dim, ql, kl
    except ValueError:
        return None


def _apply(x, layout, h_dim):
    """The oracle applied through our [outer, seq, heads, dim] reading of x."""
    y, _ = ora.fused_rope_forward(x.reshape(layout), None, head_dim=h_dim)
    return y.reshape(x.shape)


dims = st.integers(1, 5)
shapes = st.one_of(
    st.tuples(st.integers(1, 6), st.sampled_from([2, 4, 6, 8, 12, 16, 24, 30])),
    st.tuples(dims, st.integers(1, 6), st.integers(1, 3), st.sampled_from([2, 4, 6, 8, 10, 16])),
    st.tuples(st.integers(1, 6), st.integers(1, 3), st.sampled_from([2, 4, 6, 8, 10, 16])))


@st.composite
def cases(draw):
    q_shape = draw(shapes)
    head_dim = draw(st.one_of(st.none(), st.sampled_from([1, 2, 3, 4, 6, 8, 16, 32])))
    kind = draw(st.sampled_from(["none", "same", "heads", "last", "seq", "seq1", "fewer"]))
    k_shape = None
    if kind != "none":
        k = list(q_shape)
        if kind == "heads" and len(k) >= 3:
            k[-2] = draw(st.integers(1, 4))
        elif kind == "last":
            k[-1] = draw(st.sampled_from([2, 4, 6, 8, 16]))
        elif kind == "seq":
            k[-3 if len(k) >= 3 else 0] = draw(st.integers(1, 7))
        elif kind == "seq1":
            k[-3 if len(k) >= 3 else 0] = 1
        elif kind == "fewer" and len(k) >= 4:
            k = k[1:]
        k_shape = tuple(k)
    return tuple(q_shape), k_shape, head_dim


@settings(max_examples=1000, deadline=None, database=None)
@given(cases())
def test_rope_layout_matches_reference_semantics(case):
    q_shape, k_shape, head_dim = case
    q, k, ref = _reference(q_shape, k_shape, head_dim)
    ours = _ours(q_shape, k_shape, head_dim)
    if ref is None:
        assert ours is None, f"reference raises, device API accepts {case}"
        return
    rq, rk = ref
    if ours is None:
        seq_axis = -3 if len(q_shape) >= 3 else 0
        k_seq = k_shape[-3 if len(k_shape) >= 3 else 0] if k_shape is not None else None
        broadcast_k = k_shape is not None and (
            (k_seq != q_shape[seq_axis] and 1 in (k_seq, q_shape[seq_axis]))
            or len(k_shape) != len(q_shape) or rk.shape != k.shape)
        # a head_dim past the last axis makes the reference broadcast a truncated second half
        # and return another shape than q's
        broadcast_q = rq.shape != q.shape
        # an odd head_dim: the reference pairs j with j + head_dim // 2 and drops or broadcasts
        # the unpaired element
        odd = (head_dim or q_shape[-1]) % 2 == 1
        assert broadcast_k or broadcast_q or odd, \
            f"device API rejects an input the reference computes: {case}"
        return
    h_dim, ql, kl = ours
    assert int(np.prod(ql)) == q.size
    np.testing.assert_array_equal(_apply(q, ql, h_dim), rq)
    if k is not None:
        assert rk.shape == k.shape and int(np.prod(kl)) == k.size
        np.testing.assert_array_equal(_apply(k, kl, h_dim), rk)
