"""The planner (`make_plan` -> `Plan`), on the CPU: loop ranges, operand kinds and windows, outputs, carried
values and their types, and the errors each rule gives, as the reference's tests/test_plan.py pins them
(:34-276). The messages are this planner's own; each test names the rule it checks. Two of the reference's
rules are TPU layouts (windows of a multiple of 128 lanes and 8 sublanes, :164-165) and don't apply to
gfx950's LDS tiles: such windows plan here (`test_gfx950_takes_windows_of_any_size`)."""

import pytest

from tests.helpers import make_kernel, spec
from tilejax_amd import KernelError, jaxlite
from tilejax_amd.plan import Kind, Window

X = spec(256, 256)
F32, BF16, I32 = jaxlite.float32, jaxlite.bfloat16, jaxlite.int32


def plan_of(source, *inputs, **namespace):
    kernel = make_kernel(source, **namespace)
    return kernel.build(kernel.signature(*(inputs or (X,))), None)[0]


def error_of(source, *inputs, **namespace) -> str:
    with pytest.raises(KernelError) as info:
        plan_of(source, *inputs, **namespace)
    return str(info.value)


def one_input(tile: str, prologue: str = "out = jnp.zeros((256, 256))", loop: str = "for i in range(0, 256, 128):"):
    """`f(x)`: the prologue line, one parallel loop, the tile's lines inside it."""
    body = "\n".join(f"        {line}" for line in tile.strip().splitlines())
    return f"def f(x):\n    {prologue}\n    {loop}\n{body}\n    return out\n"


def reduction(before: str, step: str, after: str = "out = out.at[i : i + 128, :].set(acc)") -> str:
    return one_input(f"{before}\nfor k in range(0, 256, 128):\n    {step}\n{after}")


W = lambda loop, offset, size: Window(loop, offset, size)  # noqa: E731 (a window with no index array)


def test_a_matmul_nest():
    p = plan_of(
        """
        def f(x, y):
            M, K = x.shape
            out = jnp.zeros((M, y.shape[1]), x.dtype)
            for i in range(0, M, 128):
                for j in range(0, 256, 128):
                    acc = jnp.zeros((128, 128))
                    for k in range(0, K, 128):
                        acc += x[i : i + 128, k : k + 128] @ y[k : k + 128, j : j + 128]
                    out = out.at[i : i + 128, j : j + 128].set(acc + x[i : i + 128, 0:128])
            return out
        """,
        spec(256, 384), spec(384, 256, dtype=BF16))
    assert [(r.var, r.count) for r in p.loops] == [("i", 2), ("j", 2), ("k", 3)] and not p.single_step
    # x and y move every step; the second read of x moves only with the output tile
    assert [(op.name, op.kind) for op in p.operands] == [("x", Kind.STREAM), ("y", Kind.STREAM), ("x2", Kind.TILE)]
    assert p.operands[0].tile.windows == (W("i", 0, 128), W("k", 0, 128))
    assert p.operands[2].tile.windows == (W("i", 0, 128), W(None, 0, 128))
    assert p.carried["acc"].shape == (128, 128) and p.carried["acc"].dtype == F32
    out = p.outputs[0]
    assert (out.shape, out.dtype, out.fill, out.value) == ((256, 256), F32, 0, ((128, 128), F32))
    assert [phase.range.var for phase in p.phases] == ["k"]


def test_kinds_and_windows_of_reads_that_never_move():
    p = plan_of(
        """
        def f(x, b, s):
            out = jnp.zeros((2, 256, 128))
            for h in range(2):
                for i in range(0, 256, 128):
                    out = out.at[h, i : i + 128, :].set(x[h, i : i + 128, :] + b[:, 128:].sum(0) + s[1, 8:16, :].sum(0))
            return out
        """,
        spec(2, 256, 128), spec(8, 256), spec(2, 16, 128))
    assert p.single_step and not p.phases
    assert [op.kind for op in p.operands] == [Kind.STREAM, Kind.ONCE, Kind.ONCE]
    assert p.operands[0].tile.windows[0] == W("h", 0, None) and p.operands[0].tile.shape == (128, 128)
    assert p.operands[1].tile.windows == (W(None, 0, 8), W(None, 128, 128))
    assert p.operands[2].tile.windows == (W(None, 1, None), W(None, 8, 8), W(None, 0, 128))


def test_a_read_before_the_reduction_moves_per_tile_and_fills_are_kept():
    p = plan_of(
        """
        def f(x):
            out = jnp.full((256, 256), -1.0, jnp.bfloat16)
            for i in range(0, 256, 128):
                with jax.named_scope("pre"):
                    t = x[i : i + 128, :] * SCALE
                for k in range(0, 256, 128):
                    t = t + x[k : k + 128, :]
                out = out.at[i : i + 128, :].set(t)
            return out
        """,
        SCALE=2.0)
    assert [op.kind for op in p.operands] == [Kind.TILE, Kind.STREAM]
    assert p.outputs[0].fill == -1.0 and p.outputs[0].dtype == BF16 and set(p.carried) == {"t"}
    assert p.constants.get("SCALE") == 2.0


def test_full_with_a_keyword_fill_takes_the_fills_type():
    p = plan_of(one_input("out = out.at[i : i + 128, :].set(x[i : i + 128, :])",
                          "out = jnp.full((256, 256), fill_value=3)"))
    assert p.outputs[0].fill == 3 and p.outputs[0].dtype == I32


@pytest.mark.parametrize("prologue,message", [
    ("out = x.T", "allocate output `out` with jnp.zeros"),
    ("out = jnp.ones((256, 256))", "allocate output `out` with jnp.zeros"),
    ("out = jnp.zeros((256, 256), 'nope')", "allocate output `out` with jnp.zeros"),
    ("out = jnp.full((256, 256), jnp.ones(()))", "allocate output `out` with jnp.zeros"),
    ("out = jnp.zeros(undefined)", "can't evaluate `undefined`"),
])
def test_outputs_are_allocated_as_zeros_or_a_fill(prologue, message):
    assert message in error_of(one_input("out = out.at[i : i + 128, :].set(1.0)", prologue))


def test_the_prologue_sees_shapes_not_data():
    source = """
        def f(x):
            n = x.sum()
            out = jnp.zeros((256, 256))
            for i in range(0, 256, 128):
                out = out.at[i : i + 128, :].set(1.0)
            return out
        """
    assert "the prologue runs on the inputs' shapes and dtypes: it can't read `x`'s data" in error_of(source)
    plan_of(source.replace("n = x.sum()", "n = x.shape[0] + x.ndim + len(x) + x.size"))


@pytest.mark.parametrize("loop,message", [
    ("for i in range(0, 256.0, 128):", "loop bounds are ints"),
    ("for i in range(0, 256, 0):", "steps by 0"),
    ("for i in range(256, 0):", "which is empty"),
    ("for i in range(0, 250, 128):", "whole number of steps"),
    ("for i in range(64, 256, 128):", "whole number of steps"),
    ("for i in range(64, 320, 128):", "start at a multiple of its step"),
])
def test_loop_ranges(loop, message):
    assert message in error_of(one_input("out = out.at[i : i + 128, :].set(1.0)", loop=loop))


@pytest.mark.parametrize("read,message", [
    ("x[i : i + 128 : 2, :]", "each index is"),
    ("x[i : 128, :]", "each index is"),
    ("x[i : i + i, :]", "each index is"),
    ("x[0 : i + 128, :]", "each index is"),
    ("x[i + 1, :]", "each index is"),
    ("x[i : i + 128.0, :]", "tile bounds are ints"),
    ("x[i : i + 0, :]", "at least one element"),
    ("x[i : i + 256, :]", "reads elements 0 to 383"),
    ("x[-1, :]", "reads elements -1 to -1"),
    ("x[i : i + 128]", "index every one of x's 2 dims"),
    ("x[0, 0]", "an index array: it must be int32, not float32"),
    ("x[i : i + 128, 0]", "integer indices go before every sliced dim"),
])
def test_input_windows(read, message):
    assert message in error_of(one_input(f"out = out.at[i : i + 128, :].set({read}.sum())"))


def test_gfx950_takes_windows_of_any_size():
    """The reference's TPU layouts (:164-165) don't bind LDS tiles: a 100-column or 4-row window plans."""
    for read in ("x[i : i + 128, 0:100]", "x[i : i + 4, :]"):
        plan_of(one_input(f"out = out.at[i : i + 128, :].set({read}.sum())"))


@pytest.mark.parametrize("store,message", [
    ("out = out.at[:, :].set(1.0)", "`i` indexes exactly one dim"),
    ("out = out.at[i : i + 128, 0:128].set(1.0)", "stored whole, with `:`"),
    ("out = out.at[i, 0].set(1.0)", "keeps at least one dim"),
    ("out = out.at[i : i + 64, :].set(1.0)", "must cover the dim of 256 exactly"),
    ("out = out.at[i : i + 128, :].set((1, 2))", "must be an array or a number, not tuple"),
    ("out = out.at[i : i + 128, :].set(jnp.ones(3))", "can't store a value of shape (3,)"),
    ("out = out.at[i : i + 128, :].set(jnp.ones((128, 256, 2)))", "can't store a value of shape (128, 256, 2)"),
])
def test_output_stores(store, message):
    assert message in error_of(one_input(store))


def test_output_loops_cover_the_dim_from_zero():
    source = one_input("out = out.at[i : i + 128, :].set(1.0)", loop="for i in range(128, 256, 128):")
    assert "must cover the dim of 256 exactly" in error_of(source)


def test_a_number_start_takes_the_type_of_the_array_it_meets():
    assert plan_of(reduction("acc = 0.0", "acc = acc + x[k : k + 128, :]")).carried["acc"].shape == (128, 256)
    p = plan_of(reduction("acc = -1e30", "acc = jnp.maximum(acc, x[k : k + 128, :].astype(jnp.bfloat16))"))
    assert p.carried["acc"].dtype == BF16  # as in Python: the number takes the tile's type


@pytest.mark.parametrize("before,step,message", [
    ("acc = 0.0", "acc = acc + 1.0", "stays a Python number through the loop's steps, so it must be an array"),
    ("acc = jnp.zeros((128, 256))", "acc = jnp.concatenate([acc, acc])", "changes shape between steps"),
    ("acc = jnp.ones((128, 1))", "acc = jnp.sum(acc, 1, keepdims=True) + x[k : k + 128, :]", "changes shape"),
    ("acc = jnp.zeros((128, 256), jnp.int32)", "acc = (acc + 1).astype(jnp.int8)", "keeps one type"),
    ("acc = jnp.zeros((128, 256), jnp.bfloat16)", "acc = acc + x[k : k + 128, :]",
     "starts with it as bfloat16[128, 256] and leaves float32[128, 256]"),
    ("acc = jnp.zeros((128, 256))", "acc = acc + 1\n    acc = acc.astype(jnp.bfloat16)", "keeps one type"),
    ("acc = jnp.zeros((128, 256))\nacc = acc.astype(jnp.int8)", "acc = acc + 1.0", "keeps one type"),
    ("acc = None\nacc = jnp.zeros((128, 256))", "acc = acc + 1.0", None),  # replaced before the loop: fine
    ("acc = jnp.zeros((128, 256))\nn = acc", "acc, n = acc + 1, n", None),  # unpacking: fine
    ("acc = jnp.zeros((128, 256))", "acc = acc + undefined", "tile code failed when traced"),
    ("acc = jnp.zeros((128, 256))", "acc = acc @ x[k : k + 128, :]", "tile code failed when traced"),
])
def test_carried_values_keep_one_type(before, step, message):
    if message is None:
        plan_of(reduction(before, step))
    else:
        assert message in error_of(reduction(before, step))


def test_what_is_read_after_a_loop_but_assigned_before_it_is_carried():
    p = plan_of(reduction("acc = jnp.zeros((128, 256))\nb = acc", "c = x[k : k + 128, :]",
                          "out = out.at[i : i + 128, :].set(c + b)"))
    assert "b" in p.carried and "acc" not in p.carried


def test_a_value_a_region_leaves_stays_an_array():
    source = one_input("""
acc = jnp.zeros((128, 256))
for k in range(0, 256, 128):
    acc = acc + x[k : k + 128, :]
acc = None
b = jnp.zeros((128, 256))
for k2 in range(0, 256, 128):
    b = b + x[k2 : k2 + 128, :]
out = out.at[i : i + 128, :].set(b)
""")
    assert "makes `acc` not an array (NoneType)" in error_of(source)


def test_nothing_carries_over_from_one_tile_to_the_next():
    error = error_of(one_input("v = w + 1\nw = x[i : i + 128, :]\nout = out.at[i : i + 128, :].set(v)"))
    assert "`w` is read before the tile assigns it" in error


def test_errors_quote_the_line():
    error = error_of(reduction("acc = jnp.zeros((128, 256))", "acc = acc + undefined"))
    assert error.splitlines()[1].strip() == "acc = acc + undefined"


def test_with_blocks_are_named_scopes():
    for opener in ("jax.named_scope(NAME_NUMBER)", "jax.named_scope('a', 'b')", "jax.default_device(None)"):
        source = one_input(f"with {opener}:\n    v = 1.0\nout = out.at[i : i + 128, :].set(v)")
        assert "only `with jax.named_scope(name):` blocks" in error_of(source, NAME_NUMBER=3)
    plan_of(one_input("with jax.named_scope(NAME):\n    v = 1.0\nout = out.at[i : i + 128, :].set(v)"), NAME="ok")
