"""Loader for tests/golden/attn_golden.npz (written by tests/golden/make_golden.py)."""
from __future__ import annotations

import os
import sys
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_golden  # noqa: E402

from zwhisper_amd.ops import AttnShape  # noqa: E402

PATH = os.path.join(HERE, "golden", "attn_golden.npz")


@dataclass
class Case:
    name: str
    shape: AttnShape
    q: np.ndarray
    k: np.ndarray
    v: np.ndarray
    expected: np.ndarray  # f64, flat [n_q][out_stride]


def load_cases() -> list[Case]:
    d = np.load(PATH, allow_pickle=False)
    cases = []
    for name in d["names"]:
        name = str(name)
        s = [int(x) for x in d[f"{name}/shape"]]
        sh = AttnShape(s[0], s[1], s[2], s[3], s[4], s[5], s[6], s[7], bool(s[9]), s[8] or None)
        if f"{name}/q" in d.files:
            q, k, v = d[f"{name}/q"], d[f"{name}/k"], d[f"{name}/v"]
        else:
            uniform, rope = (bool(x) for x in d[f"{name}/flags"])
            case = {"shape": sh, "seed": int(d[f"{name}/seed"][0])}
            if uniform:
                case["dist"] = "uniform"
            if rope:
                case["rope"] = True
            q, k, v = make_golden.gen_inputs(case)
            if make_golden.digest(q, k, v) != str(d[f"{name}/sha256"]):
                raise AssertionError(f"regenerated inputs of {name} do not match the fixture checksum")
        cases.append(Case(name, sh, q, k, v, d[f"{name}/expected"]))
    return cases


def head_columns_mask(sh: AttnShape) -> np.ndarray:
    """Boolean mask over a flat out array: True where the call writes (each row's n_head*d columns)."""
    n = sh.out_len()
    m = np.zeros(max(n, 1), dtype=bool)
    for i in range(sh.n_q):
        m[i * sh.out_stride: i * sh.out_stride + sh.n_head * sh.d] = True
    return m
