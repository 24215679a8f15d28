"""Loop nests of every form the backend lowers, each with a float64 closed form of its result: tile and step
masks around an outer loop with two outputs, a mask alone, a tile mask on the only loop, single-step tiles,
per-tile reads with carried casts, broadcast stores, offset windows, a number starting a carried value, phases
back to back, unpacked carried values, partial updates of a carried array, per-tile windows shared by
consecutive tiles, and a loop that reads no input. They follow the semantics the reference's
tests/test_codegen.py pins (:31-62, 64-101, 104-123, 126-171, 174-190, 562-574, 669-689, 692-719, 722-747,
750-773, 433-452); the nests and closed forms here are this repository's. tests/test_codegen_cases.py runs
them through `kernel.reference` and builds their kernels on the CPU; tests/test_gpu_codegen_cases.py runs the
kernels on the GPU."""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Any, Callable, Dict, Tuple

import numpy as np
import torch

from tests.helpers import rand
from tilejax_amd.jaxlite import jax


def f64(t: Any) -> np.ndarray:
    return np.asarray(torch.as_tensor(t).double())


@dataclass
class Case:
    name: str
    source: str
    inputs: Callable[[], Tuple[torch.Tensor, ...]]
    want: Callable[..., Tuple[np.ndarray, ...]]
    rtol: Any = 1e-5  # per output, or one for all
    atol: Any = 1e-5
    namespace: Dict[str, Any] = field(default_factory=dict)


def _masks_want(x, y):
    xf, yf = f64(x), f64(y)
    out = np.full((4, 512, 256), -np.inf)
    other = np.zeros((4, 512, 256))
    for i in range(0, 512, 128):
        for j in range(0, 256, 128):
            if j > i:
                continue
            ks = [k for k in range(0, 384, 128) if i - 128 <= k <= i + 128]
            acc = sum(xf[:, i:i + 128, k:k + 128] @ yf[k:k + 128, j:j + 128] for k in ks)
            out[:, i:i + 128, j:j + 128] = acc
            other[:, i:i + 128, j:j + 128] = acc * 2
    return out, other


MASKS = Case("tile and step masks, an outer loop, two outputs", """
def masks(x, y):
    out = jnp.full((4, 512, 256), -jnp.inf)
    other = jnp.zeros((4, 512, 256), jnp.bfloat16)
    for b in range(4):
        for i in range(0, 512, 128):
            for j in range(0, 256, 128):
                if j > i:
                    continue
                acc = jnp.zeros((128, 128))
                for k in range(0, 384, 128):
                    if k > i + 128 or k < i - 128:
                        continue
                    acc += x[b, i : i + 128, k : k + 128] @ y[k : k + 128, j : j + 128]
                out = out.at[b, i : i + 128, j : j + 128].set(acc)
                other = other.at[b, i : i + 128, j : j + 128].set((acc * 2).astype(jnp.bfloat16))
    return out, other
""", lambda: (rand((4, 512, 384)), rand((384, 256), 1)), _masks_want, rtol=(1e-4, 1e-2), atol=(1e-3, 1e-2))

STEP_MASK = Case("a step mask alone", """
def step_mask(x):
    out = jnp.zeros((256, 128))
    for i in range(0, 256, 128):
        acc = jnp.zeros((128, 128))
        for k in range(0, 512, 128):
            if k % 256:
                continue
            acc += x[i : i + 128, k : k + 128]
        out = out.at[i : i + 128, :].set(acc)
    return out
""", lambda: (rand((256, 512)),), lambda x: (f64(x)[:, :128] + f64(x)[:, 256:384],))

TILE_MASK = Case("a tile mask on the only loop", """
def tile_mask(x):
    out = jnp.zeros((512, 128))
    for i in range(0, 512, 128):
        if i == 256:
            continue
        out = out.at[i : i + 128, :].set(x[i : i + 128, :] * 2)
    return out
""", lambda: (rand((512, 128)),), lambda x: (np.concatenate([2 * f64(x)[:256], np.zeros((128, 128)), 2 * f64(x)[384:]]),))


def _gelu(v):  # the tanh form, jax.nn.gelu's default
    return 0.5 * v * (1 + np.tanh(math.sqrt(2 / math.pi) * (v + 0.044715 * v ** 3)))


def _single_want(x, w, bias, r):
    h = f64(x) @ f64(w)
    out = np.empty((256, 256))
    for j in (0, 128):
        out[:, j:j + 128] = _gelu(h[:, j:j + 128] + f64(bias)[:, :128]) + f64(r)[:, j:j + 128] + j
    return (out,)


SINGLE_STEP = Case("single-step tiles: a product, an activation, per-tile reads and a loop value", """
def single_step(x, w, bias, r):
    out = jnp.zeros((256, 256))
    for i in range(0, 256, 128):
        for j in range(0, 256, 128):
            for k in range(0, 256, 256):
                h = x[i : i + 128, k : k + 256] @ w[k : k + 256, j : j + 128]
            h = jax.nn.gelu(h + bias[0:1, :128])
            out = out.at[i : i + 128, j : j + 128].set(h + r[i : i + 128, j : j + 128] + j)
    return out
""", lambda: (rand((256, 256)), rand((256, 256), 1) / 16, rand((1, 128), 2), rand((256, 256), 3)), _single_want,
    rtol=1e-4, atol=1e-4)


def _casts_want(x, y, r):
    acc = f64(x) @ f64(y)  # bf16 operands, f32 accumulation
    return ((acc * 2) + (acc + f64(r)),)


PER_TILE_CASTS = Case("a per-tile read, a number starting the accumulator, values renamed after the loop", """
def per_tile(x, y, r):
    out = jnp.zeros((256, 256))
    for i in range(0, 256, 128):
        for j in range(0, 256, 128):
            acc = 0.0
            first = r[i : i + 128, j : j + 128]
            t = 0.0
            for k in range(0, 384, 128):
                with jax.named_scope("dot"):
                    acc += x[i : i + 128, k : k + 128] @ y[k : k + 128, j : j + 128]
                t = acc
            acc = acc * 2
            t = t + first
            out = out.at[i : i + 128, j : j + 128].set((acc + t).astype(jnp.bfloat16))
    return out
""", lambda: (rand((256, 384), 0, torch.bfloat16), rand((384, 256), 1, torch.bfloat16), rand((256, 256), 2)),
    _casts_want, rtol=1e-2, atol=0.25)


def _ints(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-4, 5, shape, generator=g).float()  # integer-valued: every sum exact in f32


BROADCAST_STORE = Case("a broadcast store of a per-head sum, a loop of one block", """
def broadcast_store(x):
    out = jnp.zeros((2, 128, 128), jnp.int32)
    for h in range(2):
        for i in range(0, 128, 128):
            out = out.at[h, :, i : i + 128].set(1 + i + x[h, 8:16, :].sum().astype(jnp.int32))
    return out
""", lambda: (_ints((2, 128, 128), 0),),
    lambda x: (np.stack([np.full((128, 128), 1 + f64(x)[h, 8:16].sum()) for h in range(2)]),), rtol=0, atol=0)

OFFSET_WINDOWS = Case("windows of a loop that starts past zero", """
def offsets(x):
    out = jnp.zeros((256, 128))
    for i in range(0, 256, 128):
        for k in range(128, 384, 128):
            t = x[i : i + 128, k : k + 128]
        out = out.at[i : i + 128, :].set(t)
    return out
""", lambda: (rand((256, 384)),), lambda x: (f64(x)[:, 256:],), rtol=0, atol=0)

INT_START = Case("an int starting a carried value that becomes a float tile", """
def int_start(x):
    out = jnp.zeros((8, 128))
    for i in range(0, 8, 8):
        acc = 0
        for k in range(0, 256, 128):
            acc = acc + x[i : i + 8, k : k + 128]
        out = out.at[i : i + 8, :].set(acc)
    return out
""", lambda: (rand((8, 256)),), lambda x: (f64(x)[:, :128] + f64(x)[:, 128:],))

BACK_TO_BACK = Case("two reductions back to back on one carried value", """
def back_to_back(x):
    out = jnp.zeros((128, 128))
    for i in range(0, 128, 128):
        a = jnp.zeros((128, 128))
        for k in range(0, 256, 128):
            a += x[i : i + 128, k : k + 128]
        for k2 in range(0, 256, 128):
            a = jnp.maximum(a, x[i : i + 128, k2 : k2 + 128])
        out = out.at[i : i + 128, :].set(a)
    return out
""", lambda: (rand((128, 256)),),
    lambda x: (np.maximum(np.maximum(f64(x)[:, :128] + f64(x)[:, 128:], f64(x)[:, :128]), f64(x)[:, 128:]),))


def _step(acc, total, tile):
    return acc + tile, total + tile.sum(axis=1, keepdims=True)


def _unpack_want(x):
    acc, total = np.zeros((128, 128)), np.zeros((128, 1))
    for k in range(3):
        tile = f64(x)[:, 128 * k:128 * (k + 1)]
        acc, total = (acc + tile) * 0.5, total + tile.sum(axis=1, keepdims=True)
    return (acc + total,)


UNPACKING = Case("carried values unpacked from a helper", """
def unpacking(x):
    out = jnp.zeros((128, 128))
    for i in range(0, 128, 128):
        acc, total = jnp.zeros((128, 128)), jnp.zeros((128, 1))
        for k in range(0, 384, 128):
            acc, total = step(acc, total, x[i : i + 128, k : k + 128])
            acc = acc * 0.5
        out = out.at[i : i + 128, :].set(acc + total)
    return out
""", lambda: (rand((128, 384)),), _unpack_want, rtol=1e-5, atol=1e-4, namespace={"step": _step})


def _parts_want(x):
    want = 2 * f64(x)
    want[:, :8] = 1
    want[:, 8:16] += 1
    want[0] = want[1]
    return (want,)


PARTIAL_UPDATES = Case("updates of parts of a carried array", """
def parts(x):
    out = jnp.zeros((4, 128, 128))
    for i in range(0, 128, 128):
        acc = jnp.zeros((4, 128, 128))
        for k in range(4):
            acc = acc.at[k].set(x[k, i : i + 128, :] * 2)
            acc = acc.at[k, 0:8, :].set(1)
            acc = acc.at[k, 8:16, :].set(acc[k, 8:16, :] + 1)
        acc = acc.at[0].set(acc[1])
        out = out.at[:, i : i + 128, :].set(acc)
    return out
""", lambda: (rand((4, 128, 128)),), _parts_want, rtol=1e-6, atol=0)


def _shared_want(x, w, u, v, ids):
    want = np.stack([f64(x)[b] @ f64(w) + f64(u)[b].sum(0) for b in range(2)])
    want += np.repeat(np.array([f64(v)[int(n)].sum() for n in ids.tolist()]), 128)[None, :, None]
    return (want,)


SHARED_WINDOWS = Case("per-tile windows consecutive tiles share (a batch's rows, an index array's element)", """
def shared(x, w, u, v, ids):
    B, M, D = x.shape
    out = jnp.zeros((B, M, D))
    for b in range(B):
        for i in range(0, M, 128):
            t = jnp.zeros((128, D)) + u[b, 0:8, :].sum(0) + v[ids[i // 128], 0:8, :].sum()
            for k in range(0, D, 128):
                t += x[b, i : i + 128, k : k + 128] @ w[k : k + 128, :]
            out = out.at[b, i : i + 128, :].set(t)
    return out
""", lambda: (rand((2, 512, 256)), rand((256, 256), 1), rand((2, 8, 256), 2), rand((3, 8, 256), 3),
              torch.tensor([2, 2, 0, 2], dtype=torch.int32)), _shared_want, rtol=1e-4, atol=1e-3)

NO_STREAM = Case("a reduction loop that reads no input", """
def no_stream(x):
    out = jnp.zeros((256, 128))
    for i in range(0, 256, 128):
        acc = x[1, :, :]
        for k in range(0, 2):
            acc = acc * 2
        acc = acc + 1
        acc = acc + 1
        out = out.at[i : i + 128, :].set(acc)
    return out
""", lambda: (rand((2, 128, 128)),), lambda x: (np.concatenate([4 * f64(x)[1] + 2] * 2),), rtol=1e-6, atol=1e-6)

EMPTY_SOURCE = """
def empty_steps(x):
    out = jnp.zeros((256, 128))
    for i in range(0, 256, 128):
        acc = jnp.full((128, 128), 2.0)
        for k in range(0, 256, 128):
            if SKIP:
                continue
            acc += x[i : i + 128, k : k + 128]
        out = out.at[i : i + 128, :].set(acc + 1)
    return out
"""


def _empty_case(skip: str) -> Case:
    def want(x):
        out = np.full((256, 128), 3.0)
        for i in (0, 128):
            for k in (0, 128):
                if not eval(skip, {"i": i, "k": k}):
                    out[i:i + 128] += f64(x)[i:i + 128, k:k + 128]
        return (out,)

    return Case(f"a mask that skips steps ({skip}): a tile of none takes one empty step",
                EMPTY_SOURCE.replace("SKIP", skip), lambda: (rand((256, 256)),), want)


EMPTY_ALL, EMPTY_TILE, EMPTY_STEP = (_empty_case(s) for s in ("True", "i == 0", "i == 128 and k == 0"))

MASKED_CARRIED = Case("values a masked loop makes for the code after it", """
def masked_carried(x):
    out = jnp.zeros((256, 128))
    for i in range(0, 256, 128):
        acc = jnp.zeros((128, 128))
        for k in range(0, 256, 128):
            if k > i:
                continue
            acc += x[i : i + 128, k : k + 128]
            twice = acc * 2
        out = out.at[i : i + 128, :].set(twice)
    return out
""", lambda: (rand((256, 256)),),
    lambda x: (2 * np.concatenate([f64(x)[:128, :128], f64(x)[128:, :128] + f64(x)[128:, 128:]]),))

CASES = [MASKS, STEP_MASK, TILE_MASK, SINGLE_STEP, PER_TILE_CASTS, BROADCAST_STORE, OFFSET_WINDOWS, INT_START,
         BACK_TO_BACK, UNPACKING, PARTIAL_UPDATES, SHARED_WINDOWS, NO_STREAM, EMPTY_ALL, EMPTY_TILE, EMPTY_STEP,
         MASKED_CARRIED]


def check(case: Case, got: Any, wants: Tuple[np.ndarray, ...]) -> None:
    gots = got if isinstance(got, tuple) else (got,)
    assert len(gots) == len(wants), f"{case.name}: {len(gots)} outputs, want {len(wants)}"
    for k, (g, w) in enumerate(zip(gots, wants)):
        rtol = case.rtol[k] if isinstance(case.rtol, tuple) else case.rtol
        atol = case.atol[k] if isinstance(case.atol, tuple) else case.atol
        close(f"{case.name} (output {k})", g, w, rtol, atol)


def close(name: str, got: Any, want: np.ndarray, rtol: float, atol: float) -> None:
    g = f64(got)
    assert g.shape == want.shape, f"{name}: shape {g.shape}, want {want.shape}"
    finite = np.isfinite(want)
    assert (g[~finite] == want[~finite]).all(), f"{name}: the fills differ"
    err = np.abs(g[finite] - want[finite])
    bound = atol + rtol * np.abs(want[finite])
    bad = err > bound
    assert not bad.any(), f"{name}: {int(bad.sum())} of {bad.size} beyond rtol {rtol} atol {atol}; max |diff| {err.max():.3g}"
    print(f"  {name}: max |diff| {err.max() if err.size else 0:.3g}", flush=True)


# (jax is referenced by the cases' sources through make_kernel's namespace)
_ = jax
