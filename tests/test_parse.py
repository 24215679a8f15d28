"""The loop-nest language's syntax rules (tilejax_amd/parse.py), each with the KernelError it raises naming
the user's line, and the tree the parser reads a nest into."""

import ast

import pytest

import tilejax_amd
from tilejax_amd import KernelError
from tilejax_amd.jaxlite import jax, jnp
from tilejax_amd.parse import Code, Reduction, RepeatLoop
from tests.helpers import make_kernel

MATMUL = """
def mm(x, y):
    M, K = x.shape
    out = jnp.zeros((M, y.shape[1]), jnp.bfloat16)
    for i in range(0, M, 128):
        for j in range(0, y.shape[1], 128):
            acc = jnp.zeros((128, 128), jnp.float32)
            for k in range(0, K, 128):
                acc += x[i : i + 128, k : k + 128] @ y[k : k + 128, j : j + 128]
            out = out.at[i : i + 128, j : j + 128].set(acc.astype(jnp.bfloat16))
    return out
"""


def test_a_nest_reads_into_parts():
    nest = make_kernel(MATMUL).nest
    assert [loop.var for loop in nest.parallel] == ["i", "j"]
    assert [type(p) for p in nest.parts] == [Code, Reduction, Code]
    assert [loop.var for loop in nest.reductions] == ["k"]
    assert [len(s) for s in nest.segments] == [1, 1]
    assert nest.stored_in == {"out": None} and list(nest.allocations) == ["out"]


def test_two_reductions_and_a_repeat_loop():
    nest = make_kernel("""
    def two(x):
        out = jnp.zeros((128, 128))
        for i in range(0, 128, 128):
            a = jnp.zeros((128, 128))
            for k in range(0, 256, 128):
                a += x[i : i + 128, k : k + 128]
            for l in range(2):
                b = a * 2
                for k2 in range(0, 256, 128):
                    b += x[i : i + 128, k2 : k2 + 128]
                a = b
            out = out.at[i : i + 128, :].set(a)
        return out
    """).nest
    assert [type(p) for p in nest.parts] == [Code, Reduction, Code, RepeatLoop, Code]
    assert [loop.var for loop in nest.reductions] == ["k", "k2"]
    assert [r.loop.var for r in nest.repeats] == ["l"]


@pytest.mark.parametrize("source, message", [
    ("""
    def f(x):
        out = jnp.zeros((4,))
        return out
    """, "there is no `for` loop"),
    ("""
    def f(x, *rest):
        out = jnp.zeros((4,))
        for i in range(4):
            out = out.at[i : i + 1].set(x[i : i + 1])
        return out
    """, "a kernel's parameters are its input arrays"),
    ("""
    def f(x):
        out = jnp.zeros((4,))
        for i in range(4):
            out = out.at[i : i + 1].set(x[i : i + 1])
        y = 1
        return out
    """, "followed by `return` of the outputs"),
    ("""
    def f(x):
        for i in range(4):
            out = out.at[i : i + 1].set(x[i : i + 1])
        return out
    """, "must be allocated before the loops"),
    ("""
    def f(x):
        out = jnp.zeros((4,))
        for i in [0, 1]:
            out = out.at[i : i + 1].set(x[i : i + 1])
        return out
    """, "loops are `for v in range"),
    ("""
    def f(x):
        out = jnp.zeros((4,))
        for i in range(4):
            if i > 2:
                out = out.at[i : i + 1].set(x[i : i + 1])
        return out
    """, "use jnp.where instead of `if`"),
    ("""
    def f(x):
        out = jnp.zeros((4,))
        for i in range(4):
            t = x
            out = out.at[i : i + 1].set(x[i : i + 1])
        return out
    """, "is an input: kernel code reads tiles of it"),
    ("""
    def f(x):
        out = jnp.zeros((4,))
        for i in range(4):
            t = out[i : i + 1]
            out = out.at[i : i + 1].set(x[i : i + 1])
        return out
    """, "output `out`'s tiles are written as"),
    ("""
    def f(x):
        out = jnp.zeros((4,))
        for i in range(4):
            out = out.at[i : i + 1].set(x[i : i + 1])
            out = out.at[i : i + 1].set(x[i : i + 1])
        return out
    """, "is stored twice in a tile"),
    ("""
    def f(x):
        out = jnp.zeros((4, 4))
        for i in range(4):
            a = jnp.zeros((1, 4))
            for k in range(4):
                a += x[i : i + 1, k : k + 1]
            b = k
            out = out.at[i : i + 1, :].set(a)
        return out
    """, "`k` is only defined inside its reduction loop"),
    ("""
    def f(x):
        out = jnp.zeros((4,))
        for i in range(4):
            i = 2
            out = out.at[i : i + 1].set(x[i : i + 1])
        return out
    """, "loop variable `i` can't be assigned"),
    ("""
    def f(x):
        out = jnp.zeros((4, 4))
        for i in range(4):
            if x > 0:
                continue
            out = out.at[i : i + 1, :].set(x[i : i + 1, :])
        return out
    """, "masks are evaluated when the kernel is built"),
    ("""
    def f(x):
        out = jnp.zeros((4,))
        for i in range(4):
            out = out.at[i : i + 1].set((y := x[i : i + 1]))
        return out
    """, "can't assign inside expressions"),
])
def test_rules(source, message):
    with pytest.raises(KernelError, match=message) as info:
        make_kernel(source)
    assert ":" in str(info.value).splitlines()[0]  # file:line: the user's line


def test_errors_quote_the_line():
    with pytest.raises(KernelError) as info:
        make_kernel("""
        def f(x):
            out = jnp.zeros((4,))
            for i in range(4):
                t = x
                out = out.at[i : i + 1].set(x[i : i + 1])
            return out
        """)
    first, quoted = str(info.value).splitlines()[:2]
    assert first.startswith("<tilejax-test-") and ":5: " in first
    assert quoted.strip() == "t = x"



# ------------------------------------------------------------------ the reference's rules, case by case
# Functions shaped as the reference's tests/test_parse.py:60-375 cases (each broken one way); the messages are
# the rule each must name.

def _f_args(x, *rest):
    pass
def _g_args(x, y=1, z=2):
    pass
def _h_args(x, *, y):
    pass
def _no_loop(x):
    return x
def _bad_prologue(x):
    if x:
        pass
    for i in range(1):
        pass
    return x
def _nothing_after(x):
    for i in range(1):
        pass
def _code_after(x):
    out = jnp.zeros(1)
    for i in range(1):
        pass
    out = out + 1
    return out
def _returns_expression(x):
    for i in range(1):
        pass
    return x + 1
def _returns_twice(x):
    out = jnp.zeros(1)
    for i in range(1):
        pass
    return out, out
def _returns_nothing(x):
    for i in range(1):
        pass
    return
def _unallocated(x):
    for i in range(1):
        pass
    return out  # noqa: F821
def _allocated_twice(x):
    out = jnp.zeros(1)
    out = jnp.zeros(2)
    for i in range(1):
        pass
    return out
def _unpacked(x):
    out, other = jnp.zeros(1), 2
    for i in range(1):
        pass
    return out
def _augmented(x):
    out = jnp.zeros(1)
    out += 1
    for i in range(1):
        pass
    return out
def _not_range(x):
    out = jnp.zeros(1)
    for i in [0, 1]:
        pass
    return out
def _keywords(x):
    out = jnp.zeros(1)
    for i in range(stop=1):
        pass
    return out
def _unpacking(x):
    out = jnp.zeros(1)
    for i, j in range(1):
        pass
    return out
def _with_else(x):
    out = jnp.zeros(1)
    for i in range(1):
        pass
    else:
        pass
    return out
def _only_a_mask(x):
    out = jnp.zeros(1)
    for i in range(1):
        if i:
            continue
    return out
def _nested_repeats(x):
    out = jnp.zeros(1)
    for i in range(1):
        for r in range(1):
            for k in range(1):
                for k2 in range(1):
                    a = 1
        out = out.at[i].set(1)
    return out
def _masked_repeat(x):
    out = jnp.zeros(1)
    for i in range(1):
        for r in range(2):
            if r:
                continue
            for k in range(1):
                a = 1
        out = out.at[i].set(1)
    return out
def _loop_in_a_scope(x):
    out = jnp.zeros(1)
    for i in range(1):
        with jax.named_scope("s"):
            for k in range(1):
                a = 1
        out = out.at[i].set(1)
    return out
def _tunable_whole(x, tiles=None):
    out = jnp.zeros((8, 128))
    for i in range(0, 8, 8):
        t = tiles
        out = out.at[i : i + 8, :].set(x[i : i + 8, :])
    return out
def _store_in_pre(x):
    out = jnp.zeros((8, 128))
    for i in range(0, 8, 8):
        out = out.at[i : i + 8, :].set(1.0)
        for k in range(1):
            a = 1
    return out
def _store_in_a_repeat_loop(x):
    out = jnp.zeros((8, 128))
    for i in range(0, 8, 8):
        a = 1
        for r in range(2):
            for k in range(1):
                out = out.at[i : i + 8, :].set(1.0)
    return out
def _stored_twice(x):
    out = jnp.zeros((8, 128))
    for i in range(0, 8, 8):
        out = out.at[i : i + 8, :].set(1.0)
        out = out.at[i : i + 8, :].set(2.0)
    return out
def _never_stored(x):
    out = jnp.zeros((8, 128))
    for i in range(0, 8, 8):
        a = 1
    return out
def _reads_an_output(x):
    out = jnp.zeros((8, 128))
    for i in range(0, 8, 8):
        out = out.at[i : i + 8, :].set(out[i : i + 8, :])
    return out
def _reads_the_reduction_variable(x):
    out = jnp.zeros((8, 128))
    for i in range(0, 8, 8):
        for k in range(1):
            a = 1
        out = out.at[i : i + 8, :].set(k)
    return out
def _reads_an_inner_loop(x):
    out = jnp.zeros((8, 128))
    for i in range(0, 8, 8):
        if j > 0:  # noqa: F821
            continue
        for j in range(0, 128, 128):
            out = out.at[i : i + 8, j : j + 128].set(1.0)
    return out
def _asserts_shapes(x):
    assert x.shape[0] == 8
    out = jnp.zeros((8, 128))
    pass
    for i in range(0, 8, 8):
        out = out.at[i : i + 8, :].set(1.0)
    return out


RULE_CASES = [
    (_f_args, "its input arrays, then optionally a tunable"), (_g_args, "its input arrays, then optionally a tunable"),
    (_h_args, "its input arrays, then optionally a tunable"), (_no_loop, "no `for` loop"),
    (_bad_prologue, "assignments and asserts"), (_nothing_after, "followed by `return`"),
    (_code_after, "followed by `return`"), (_returns_expression, "return the outputs by name"),
    (_returns_nothing, "return the outputs by name"), (_returns_twice, "returned once"),
    (_unallocated, "must be allocated before the loops"), (_allocated_twice, "allocate output `out` once"),
    (_unpacked, "allocate output `out` once"), (_augmented, "allocate output `out` once"),
    (_not_range, "`for v in range(start, stop, step)`"), (_keywords, "`for v in range(start, stop, step)`"),
    (_unpacking, "`for v in range(start, stop, step)`"), (_with_else, "`else` block"),
    (_only_a_mask, "nothing to run"), (_nested_repeats, "repeat loops don't nest"),
    (_masked_repeat, "a repeat loop (around reduction loops) can't be masked"),
    (_loop_in_a_scope, "loops nest only as parallel loops around reduction (and repeat) loops"),
    (_tunable_whole, "`tiles` is the kernel's tunable: tile code reads its fields"),
    (_store_in_pre, "after the reduction loop"), (_store_in_a_repeat_loop, "in the body of a reduction loop"),
    (_stored_twice, "stored twice"), (_never_stored, "no tile stores output `out`"),
    (_reads_an_output, "tiles can't be read"), (_reads_the_reduction_variable, "only defined inside its reduction loop"),
    (_reads_an_inner_loop, "not `j`"), (len, "can't read its source"), (lambda x: x, "defined with `def`"),
]


@pytest.mark.parametrize("fn,message", RULE_CASES, ids=lambda v: getattr(v, "__name__", None) if callable(v) else None)
def test_each_rule_names_itself(fn, message):
    with pytest.raises(KernelError) as info:
        tilejax_amd.kernel(fn)
    assert message in str(info.value)


def test_asserts_in_the_prologue():
    assert isinstance(tilejax_amd.kernel(_asserts_shapes).nest.prologue[0], ast.Assert)
