"""The loop-nest language's syntax rules (tilejax_amd/parse.py), each with the KernelError it raises naming
the user's line, and the tree the parser reads a nest into."""

import pytest

from tilejax_amd import KernelError
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
