"""The host-side API, on the CPU: what `lower` describes and caches, input and tunable errors, `compare`'s
tolerances, tunables and neighbours, and `@`'s semantics in `kernel.fn` (the reference's tests/test_api.py
and tests/test_tunable.py, for the behaviour this package mirrors)."""

import dataclasses

import pytest
import torch

import tilejax_amd as autokernel
from examples.matmul import MatmulTiles, matmul
from tilejax_amd import KernelError, jaxlite
from tilejax_amd.api import compare
from tilejax_amd.pipeline import Pipeline
from tilejax_amd.tunable import choices, is_tunable, neighbours

F32 = jaxlite.float32
TILES = MatmulTiles(tm=128, tn=128, tk=128)


def test_lowered_describes_the_kernel():
    lowered = matmul.lower(((256, 384), F32), ((384, 256), F32), TILES)
    assert (lowered.steps, lowered.tiles, lowered.total_tiles) == (12, 4, 4)  # test_api.py:20-30
    assert str(lowered.pipeline) == f"{lowered.pipeline.input_buffers} input / 2 output buffers"
    assert lowered.config.tunable == TILES and str(lowered.config).startswith("MatmulTiles(tm=128")
    assert matmul.lower(((256, 384), F32), ((384, 256), F32), TILES) is lowered  # built once per signature
    assert repr(matmul) == "<tilejax_amd.Kernel matmul>" and matmul.__name__ == "matmul"
    assert matmul.source(((256, 384), F32), ((384, 256), F32), TILES) == lowered.source


def test_inputs_are_arrays_of_the_right_count():
    x = torch.randn(256, 256)
    with pytest.raises(KernelError, match=r"takes 2 input arrays \(x, y\), then optionally `tiles`; got 1"):
        matmul(x)
    with pytest.raises(KernelError, match="input `y` must be an array, got float"):
        matmul(x, 1.0)
    with pytest.raises(KernelError, match="`tiles` must be a MatmulTiles, not tuple"):
        matmul(x, x, (128, 128, 128))


def test_compare_tolerances():
    a = torch.tensor([1.0, 2.0, float("nan"), float("inf")])
    assert compare("f32", a, a) == 0.0
    assert compare("f32", a + torch.tensor([1e-5, 0, 0, 0]), a) == pytest.approx(1e-5, rel=1e-2)
    with pytest.raises(AssertionError, match="1 of 4 elements"):
        compare("f32", a + torch.tensor([1.0, 0, 0, 0]), a)
    b = torch.tensor([100.0, 1.0], dtype=torch.bfloat16)
    assert compare("bf16", b + torch.tensor([0, 1.0], dtype=torch.bfloat16), b) == 1.0  # 2e-2 of the largest
    i = torch.tensor([1, 2], dtype=torch.int32)
    with pytest.raises(AssertionError):
        compare("i32", i + 1, i)
    assert compare("i32", i, i) == 0.0


@autokernel.tunable
class Tiles:
    tm: int = autokernel.choice(128, 256, 512, default=256)
    tk: int = autokernel.choice(128, 256)


def test_a_tunable_is_a_frozen_dataclass_of_choices():
    t = Tiles()
    assert (t.tm, t.tk) == (256, 128) and is_tunable(t) and not is_tunable(3) and not is_tunable(Tiles)
    with pytest.raises(dataclasses.FrozenInstanceError):
        t.tm = 512  # type: ignore[misc]
    assert hash(t) == hash(Tiles())
    assert choices(t) == {"tm": (128, 256, 512), "tk": (128, 256)}


def test_neighbours_move_one_field_one_step():
    assert list(neighbours(Tiles())) == [Tiles(tm=512), Tiles(tm=128), Tiles(tk=256)]  # test_tunable.py:28-30
    assert list(neighbours(Tiles(tm=384))) == [Tiles(tm=384, tk=256)]  # a value off the choices stays put


def test_fields_must_be_choices():
    with pytest.raises(TypeError, match=r"autokernel\.choice|choice"):

        @autokernel.tunable
        class Bad:
            tm: int = 128

    with pytest.raises(ValueError, match="at least one value"):
        autokernel.choice()
    with pytest.raises(ValueError, match="isn't one of the choices"):
        autokernel.choice(1, 2, default=3)


def test_pipelines_are_checked():
    with pytest.raises(KernelError, match="1 to 4 input buffers"):
        Pipeline(5, 2)
    with pytest.raises(KernelError, match="1 to 3 output buffers"):
        Pipeline(2, 0)


def test_fn_multiplies_bf16_with_f32_accumulation():
    """`@` in `kernel.fn` (the reference's mxu.py:21-43): bf16 operands, f32 products and sums, the tile
    cast back at the store; the same as float64 to f32 rounding."""
    g = torch.Generator().manual_seed(0)
    x, y = torch.randn(256, 256, generator=g).bfloat16(), torch.randn(256, 256, generator=g).bfloat16()
    got = matmul.fn(x, y, TILES)
    want = (x.double() @ y.double()).bfloat16()
    assert got.dtype == torch.bfloat16
    assert (got.float() - want.float()).abs().max().item() <= 2e-2 * want.float().abs().max().item()


def test_compare_checks_a_big_output_a_chunk_at_a_time(monkeypatch):
    """The reference's tests/test_api.py:103-108: the bf16 floor is 2e-2 of the largest value anywhere, even
    when it sits in a later chunk."""
    from tilejax_amd import api

    monkeypatch.setattr(api, "COMPARE_CHUNK", 2)
    want = torch.tensor([[1.0, 2.0, 3.0], [4.0, 5.0, 100.0]], dtype=torch.bfloat16)
    one = want.clone()
    one[0, 0] += 1.0
    assert compare("bf16", one, want) == 1.0
    two = want.clone()
    two[0, 0] += 4.0
    two[1, 1] -= 4.0
    with pytest.raises(AssertionError, match="2 of 6 elements"):
        compare("bf16", two, want)


SCALED = """
def scaled(x):
    out = jnp.zeros(x.shape)
    for i in range(0, x.shape[0], 8):
        out = out.at[i : i + 8, :].set(x[i : i + 8, :] * SCALE)
    return out
"""


def test_constants_are_read_when_a_signature_is_first_built():
    """As jax.jit reads globals when it traces: a signature built before a global changes keeps the value it
    read; a new signature reads the new one (the reference's tests/test_api.py:55-62)."""
    from tests.helpers import make_kernel, rand

    kernel = make_kernel(SCALED, SCALE=2.0)
    x = rand((8, 128))
    first = kernel.reference(x)
    kernel.fn.__globals__["SCALE"] = 3.0
    assert torch.equal(kernel.reference(x), first)
    wide = rand((16, 128))
    assert torch.allclose(kernel.reference(wide), 3 * wide)


def test_closures_are_read_too():
    from tests.helpers import rand
    from tilejax_amd.jaxlite import jnp

    def make(scale):
        @autokernel.kernel
        def scaled(x):
            out = jnp.zeros(x.shape)
            for i in range(0, x.shape[0], 8):
                out = out.at[i : i + 8, :].set(x[i : i + 8, :] * scale)
            return out

        return scaled

    x = rand((16, 128))
    assert torch.allclose(make(4.0).reference(x), 4 * x) and torch.allclose(make(0.5).reference(x), x / 2)


def test_errors_quote_the_line_when_they_can():
    import ast

    node = ast.Pass(lineno=1)
    assert str(KernelError("boom", filename=__file__, node=node)).startswith(f"{__file__}:1: boom\n    ")
    assert str(KernelError("boom", filename="<nowhere>", node=node)) == "<nowhere>:1: boom"
    assert str(KernelError("boom")) == "boom"


def test_matmul_assignment():
    """`acc @= w[k]` on a carried value (the reference's tests/test_api.py:164-180)."""
    from tests.helpers import make_kernel, rand

    kernel = make_kernel("""
    def f(x, w):
        out = jnp.zeros((128, 128))
        for i in range(0, 128, 128):
            acc = x[i : i + 128, :]
            for k in range(0, 2):
                acc @= w[k, :, :]
            out = out.at[i : i + 128, :].set(acc)
        return out
    """)
    x, w = rand((128, 128)), rand((2, 128, 128), 1) / 8
    want = x.double() @ w[0].double() @ w[1].double()
    assert (kernel.reference(x, w).double() - want).abs().max() < 1e-4
    assert kernel.lower(x, w).program.notes["family"] == "generic"


def test_prologue_comprehensions_see_globals():
    from tests.helpers import make_kernel, spec

    kernel = make_kernel("""
    def f(x):
        R = min(d // T for d in x.shape)
        out = jnp.zeros((R * T, 128))
        for i in range(0, R * T, T):
            out = out.at[i : i + T, :].set(x[i : i + T, :])
        return out
    """, T=8)
    assert kernel.lower(spec(16, 128)).tiles == 2
