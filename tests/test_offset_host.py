"""CPU checks behind the GPU tests of data away from the origin (tests/test_offset_gpu.py).

* The plain fp32 norm form ||q||^2 + ||x||^2 - 2 q.x, replayed in numpy, loses the true
  neighbours on those inputs; so the GPU tests fail unless the GPU path really corrects for it.
* The selection error bound the GPU path relies on (|GEMM-form score - exact distance| <=
  c (||q'|| + ||x'||)^2 with c = 1.02 (2 gamma_{D+2} + 4u), u = 2^-24, for operands shifted by the
  column means) holds for sequential fp32 evaluation on adversarial inputs, and the column-mean
  shift is what makes it small.
"""
import numpy as np

U = 2.0 ** -24


def gamma(n):
    return n * U / (1 - n * U)


def l2_coeff(d):
    return 1.02 * (2 * gamma(d + 2) + 4 * U)


def norm_form_f32(q, x):
    """fp32 ||q||^2 + ||x||^2 - 2 q.x with float32 BLAS products (the GEMM form)."""
    q = q.astype(np.float32)
    x = x.astype(np.float32)
    qn = np.einsum("ij,ij->i", q, q, dtype=np.float32)
    xn = np.einsum("ij,ij->i", x, x, dtype=np.float32)
    return np.maximum(qn[:, None] + (xn[None, :] - np.float32(2) * (q @ x.T)), np.float32(0))


def exact_l2(q, x):
    q = q.astype(np.float64)
    x = x.astype(np.float64)
    return ((q[:, None, :] - x[None, :, :]) ** 2).sum(-1)


def recall(sel, exact, k):
    kth = np.sort(exact, 1)[:, k - 1:k]
    got = np.argsort(sel, 1, kind="stable")[:, :k]
    return float(np.mean(np.take_along_axis(exact, got, 1) <= kth * (1 + 1e-6)))


def far_clusters(n_clusters, per, dim, seed, spread=1000.0, noise=0.01):
    rng = np.random.default_rng(seed)
    centres = rng.standard_normal((n_clusters, dim)) * spread
    lab = np.repeat(np.arange(n_clusters), per)
    return (centres[lab] + rng.standard_normal((n_clusters * per, dim)) * noise).astype(np.float32), centres


def test_plain_norm_form_fails_on_offset_data():
    rng = np.random.default_rng(0)
    x = (1000 + rng.standard_normal((4000, 128))).astype(np.float32)
    q = (1000 + rng.standard_normal((20, 128))).astype(np.float32)
    ex = exact_l2(q, x)
    assert recall(norm_form_f32(q, x), ex, 10) < 0.5
    # centring by the column means restores the ranking on this data
    mu = x.mean(0, dtype=np.float64).astype(np.float32)
    assert recall(norm_form_f32(q - mu, x - mu), ex, 10) > 0.99


def test_centring_is_not_enough_for_far_tight_clusters():
    """The direct-form fallback case: even centred, the norm form cannot rank members of one
    tight cluster, and the error bound covers the whole cluster."""
    x, centres = far_clusters(20, 200, 64, 7)
    rng = np.random.default_rng(8)
    q = (centres[rng.integers(0, 20, 10)] + rng.standard_normal((10, 64)) * 0.01).astype(np.float32)
    mu = x.mean(0, dtype=np.float64).astype(np.float32)
    ex = exact_l2(q, x)
    assert recall(norm_form_f32(q - mu, x - mu), ex, 10) < 0.9
    qs, xs = (q - mu).astype(np.float64), (x - mu).astype(np.float64)
    e = l2_coeff(64) * (np.linalg.norm(qs, axis=1) + np.linalg.norm(xs, axis=1).max()) ** 2
    kth = np.sort(ex, 1)[:, 9]
    within = (ex <= (kth + 2 * e)[:, None]).sum(1)
    assert np.all(within >= 200)  # the whole cluster: more than the margin of 16-256 kept entries


def _seq_dot_f32(a, b):
    """Left-to-right fp32 sum of products (each step rounded)."""
    acc = np.zeros(a.shape[0], np.float32)
    for i in range(a.shape[1]):
        acc = (acc + a[:, i] * b[:, i]).astype(np.float32)
    return acc


def test_selection_error_bound_holds():
    """Worst-ish cases for the shifted norm form: large shared offsets, mixed signs, and
    near-duplicates, evaluated with sequential fp32 sums.  The observed error must stay under the
    bound, and the bound must be tight enough to be useful (within 1e3 of the observed maximum)."""
    rng = np.random.default_rng(3)
    worst = 0.0
    for d, off, scale in [(128, 1000.0, 1.0), (96, 0.0, 50.0), (768, 10.0, 1.0), (32, 1e4, 3.0)]:
        x = (off + scale * rng.standard_normal((300, d))).astype(np.float32)
        q = np.concatenate([x[:100] + np.float32(1e-3) * rng.standard_normal((100, d)).astype(np.float32),
                            (off + scale * rng.standard_normal((100, d))).astype(np.float32)])
        mu = x.mean(0, dtype=np.float64).astype(np.float32)
        xs = (x - mu).astype(np.float32)
        qs = (q - mu).astype(np.float32)
        xn = _seq_dot_f32(xs, xs)
        qn = _seq_dot_f32(qs, qs)
        pairs = rng.integers(0, 300, 200)
        dots = _seq_dot_f32(qs, xs[pairs])
        s = (qn + (xn[pairs] - np.float32(2) * dots).astype(np.float32)).astype(np.float32)
        true = ((q.astype(np.float64) - x[pairs].astype(np.float64)) ** 2).sum(1)
        bound = l2_coeff(d) * (np.linalg.norm(qs.astype(np.float64), axis=1) +
                               np.linalg.norm(xs[pairs].astype(np.float64), axis=1)) ** 2
        err = np.abs(s.astype(np.float64) - true)
        assert np.all(err <= bound), (d, off, float((err / bound).max()))
        worst = max(worst, float((err / bound).max()))
    assert worst > 1e-3
