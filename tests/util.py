"""Small numpy helpers shared by the tests."""
import numpy as np


def bits(a):
    a = np.asarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


def same(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    return a.shape == b.shape and np.array_equal(bits(a), bits(b))


def first_diff(a, b):
    d = np.flatnonzero(bits(np.ravel(a)) != bits(np.ravel(b)))
    if d.size == 0:
        return None
    i = int(d[0])
    return i, float(np.ravel(a)[i]), float(np.ravel(b)[i]), int(d.size)
