"""Synthetic workloads of the benchmark configurations, with a fixed draw order.

The reference defines no scripts for these shapes, so the seeding and draw
order below is this package's manifest (every tensor comes from the
reference's generator via rustgears_amd.rng, in this order):

  quickstart  manual_seed(42); Linear(4,32) [kaiming W, bias]; BatchNorm1d(32);
              Linear(32,3); BN stats (running_mean = normal*0.1, then
              running_var = U(0.5,1.5), per BN in order); x = randn[64,4]
  deep_mlp    manual_seed(1); Linear 784->1024, BN1d, ReLU, 1024->1024, BN1d, ReLU,
              1024->10 (kaiming + bias); BN stats as above; x = rand[rows,784]
  cnn         manual_seed(7); Conv 3->32 k3 p1, BN2d, ReLU, MaxPool 2, Conv 32->64
              k3 p1, BN2d, ReLU, MaxPool 2, Flatten, Linear 4096->256, ReLU,
              Linear 256->10; BN stats; x = randn[n,3,32,32]
  linear_stack manual_seed(3); depth x (Linear.xavier(w,w) + GELU);
              x = randn[rows, w]
  gemv        manual_seed(5); Linear.xavier(d,h) + SiLU (extension activation),
              Linear.xavier(h,d); x = randn[batch, d]
  (Linear.xavier draws xavier_uniform W [in,out] then bias_uniform [out].)
Every builder takes size arguments so tests can run the same recipe small.
"""
from __future__ import annotations

from typing import List, Tuple

import numpy as np

from . import nn, rng
from .inference import Activation, LayerSpec


def set_bn_stats(bns) -> None:
    for bn in bns:
        bn.running_mean = nn.normal([bn.num_features], 0.1)
        bn.running_var = rng.uniform([bn.num_features], 0.5, 1.5)


def quickstart(rows: int = 64, seed: int = 42) -> Tuple[nn.Sequential, np.ndarray]:
    rng.manual_seed(seed)
    l1 = nn.Linear(4, 32)
    bn = nn.BatchNorm1d(32)
    l2 = nn.Linear(32, 3)
    model = nn.Sequential().add(l1).add(bn).add(nn.Relu()).add(l2)
    set_bn_stats([bn])
    x = rng.randn([rows, 4])
    return model, x


def deep_mlp(rows: int = 4096, d_in: int = 784, hidden: int = 1024, d_out: int = 10,
             seed: int = 1) -> Tuple[nn.Sequential, np.ndarray]:
    rng.manual_seed(seed)
    l1, bn1 = nn.Linear(d_in, hidden), nn.BatchNorm1d(hidden)
    l2, bn2 = nn.Linear(hidden, hidden), nn.BatchNorm1d(hidden)
    l3 = nn.Linear(hidden, d_out)
    model = (nn.Sequential().add(l1).add(bn1).add(nn.Relu()).add(l2).add(bn2).add(nn.Relu()).add(l3))
    set_bn_stats([bn1, bn2])
    x = rng.rand([rows, d_in])
    return model, x


def cnn(n: int = 256, hw: int = 32, c1: int = 32, c2: int = 64, fc: int = 256, classes: int = 10,
        seed: int = 7) -> Tuple[nn.Sequential, np.ndarray]:
    rng.manual_seed(seed)
    conv1, bn1 = nn.Conv2d(3, c1, 3).padding(1), nn.BatchNorm2d(c1)
    conv2, bn2 = nn.Conv2d(c1, c2, 3).padding(1), nn.BatchNorm2d(c2)
    flat = c2 * (hw // 4) * (hw // 4)
    fc1, fc2 = nn.Linear(flat, fc), nn.Linear(fc, classes)
    model = (nn.Sequential().add(conv1).add(bn1).add(nn.Relu()).add(nn.MaxPool2d(2))
             .add(conv2).add(bn2).add(nn.Relu()).add(nn.MaxPool2d(2)).add(nn.Flatten())
             .add(fc1).add(nn.Relu()).add(fc2))
    set_bn_stats([bn1, bn2])
    x = rng.randn([n, 3, hw, hw])
    return model, x


def linear_stack(rows: int = 8192, width: int = 4096, depth: int = 4,
                 seed: int = 3) -> Tuple[nn.Sequential, np.ndarray]:
    rng.manual_seed(seed)
    model = nn.Sequential()
    for _ in range(depth):
        model.add(nn.Linear.xavier(width, width)).add(nn.Gelu())
    x = rng.randn([rows, width])
    return model, x


def gemv(batch: int = 1, d: int = 8192, h: int = 28672, seed: int = 5,
         act: Activation = Activation.SILU) -> Tuple[List, np.ndarray]:
    rng.manual_seed(seed)
    l1 = nn.Linear.xavier(d, h)
    l2 = nn.Linear.xavier(h, d)
    layers = l1.export() + [LayerSpec.Activation(act)] + l2.export()
    x = rng.randn([batch, d])
    return layers, x


def macs(name: str, **kw) -> int:
    """2 x MACs = ops; MAC formulas of npu.rs:309 (rows*in*out) and :328."""
    if name == "linear_stack":
        rows, w, depth = kw.get("rows", 8192), kw.get("width", 4096), kw.get("depth", 4)
        return rows * w * w * depth
    if name == "gemv":
        b, d, h = kw.get("batch", 1), kw.get("d", 8192), kw.get("h", 28672)
        return b * d * h * 2
    raise KeyError(name)
