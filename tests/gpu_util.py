"""Helpers for the GPU parity tests: seeded inputs (the library's counter-based generator),
oracle-quantised weights, and host <-> device copies through torch."""
import numpy as np
import torch

import oracle as O
import q35


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def normal(stream, shape, sigma=1.0, seed=0):
    n = int(np.prod(shape))
    return q35.synth_normal(seed, stream, n, sigma).reshape(shape)


def q8(stream, rows, cols, sigma=0.02, seed=0):
    """(oracle Q8Mat, device Q8FTensor pair maker) for an f32 N(0, sigma) matrix [rows][cols]."""
    W = O.quantize(normal(stream, (rows, cols), sigma, seed))
    return W


def q8_dev(W, layout):
    return q35.Q8FTensor(dev(W.q), dev(W.s), layout)
