"""Synthetic inputs: the host twin of glt_fill_normal.

Value i of tensor (seed, tensor_id) is
    key  = splitmix64(seed ^ splitmix64(tensor_id + 0x632BE59BD9B4E019))
    r1, r2 = splitmix64(key + 2p), splitmix64(key + 2p + 1),  p = i // 2
    u1 = ((r1 >> 11) + 1) * 2^-53,  u2 = (r2 >> 11) * 2^-53
    z  = sqrt(-2 ln u1) * (cos if i even else sin)(2 pi u2)      (f64)
    out = f32(mean + std * z)  [-> RNE bf16]
so a host check and a GPU run can draw the same tensor. The f64
transcendental functions of numpy and the device library may differ in the
last bit, which after rounding to f32 changes a value only rarely; parity
tests therefore upload host-drawn inputs.
"""
import numpy as np

M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def splitmix64(x):
    x = np.asarray(x, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def tensor_key(seed, tensor_id):
    inner = splitmix64(np.uint64(tensor_id) + np.uint64(0x632BE59BD9B4E019))
    return splitmix64(np.uint64(seed) ^ inner)


def normal(shape, seed, tensor_id, mean=0.0, std=1.0, start=0):
    """float32 array of the given shape; element i of the flat tensor is value
    start + i of the (seed, tensor_id) stream."""
    n = int(np.prod(shape))
    key = tensor_key(seed, tensor_id)
    idx = np.arange(start, start + n, dtype=np.uint64)
    p = idx >> np.uint64(1)
    with np.errstate(over="ignore"):
        r1 = splitmix64(key + np.uint64(2) * p)
        r2 = splitmix64(key + np.uint64(2) * p + np.uint64(1))
    u1 = ((r1 >> np.uint64(11)) + np.uint64(1)).astype(np.float64) * 2.0 ** -53
    u2 = (r2 >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    rad = np.sqrt(-2.0 * np.log(u1))
    th = 6.283185307179586 * u2
    z = np.where((idx & np.uint64(1)) == 0, rad * np.cos(th), rad * np.sin(th))
    return (mean + std * z).astype(np.float32).reshape(shape)


# Seeds and tensor ids of the synthetic workloads: base weights seed 0,
# x seed 100, dy seed 200, RMSNorm gamma seed 300, graft slice k seed k.
SEED_BASE, SEED_X, SEED_DY, SEED_GAMMA = 0, 100, 200, 300
TID_GATE, TID_UP, TID_DOWN = 1, 2, 3
TID_X, TID_DY, TID_GAMMA = 10, 11, 12
