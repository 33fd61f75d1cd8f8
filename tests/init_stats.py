"""Distribution checks for weight-initialisation draws (shared by the CPU
init tests and the GPU tests of constructed layers).

check_uniform: every value in [lo, hi], both ends reached within 25/n of
the span (a correct draw misses with probability ~e^-25), mean and mean
squared deviation within 6 sigma of U(lo, hi)'s.  check_normal: mean and
mean squared deviation within 6 sigma of N(mean, sd)'s.
"""
import numpy as np


def check_uniform(w, lo, hi):
    n = w.size
    assert w.min() >= lo and w.max() <= hi, (w.min(), w.max(), lo, hi)
    span = hi - lo
    assert w.min() <= lo + 25.0 / n * span and w.max() >= hi - 25.0 / n * span, \
        f"support not reached: [{w.min()}, {w.max()}] vs [{lo}, {hi}]"
    mu, var = (lo + hi) / 2, span * span / 12
    assert abs(w.mean() - mu) <= 6 * np.sqrt(var / n)
    # Var((x-mu)^2) for a uniform = span^4/80 - var^2
    d2 = (w - mu) ** 2
    assert abs(d2.mean() - var) <= 6 * np.sqrt((span ** 4 / 80 - var * var) / n)


def check_normal(w, mean, sd):
    n = w.size
    assert abs(w.mean() - mean) <= 6 * sd / np.sqrt(n)
    # Var((x-mu)^2) for a normal = 2 sd^4
    d2 = (w - mean) ** 2
    assert abs(d2.mean() - sd * sd) <= 6 * np.sqrt(2.0 / n) * sd * sd
