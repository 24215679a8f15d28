"""Grouped matmul with runtime expert windows: each group of G rows of `xs` through its expert's weights.

The spec of BASELINE.json config 4, in the form the reference's grouped kernels take
(examples/moe.py:167-187 `expert_ffn`: the runtime mask `tile_expert[i // G] < 0` and the runtime window
`w[tile_expert[i // G], ...]`; the single-matrix grouped form of tests/test_index_arrays.py:109-125):
tokens arrive sorted by expert in groups of G rows, `group_expert[g]` names group g's expert (or -1 for an
unused group, whose rows stay zero), and the window `w[group_expert[i // G], k : k + tk, j : j + tn]` is
chosen on the device. Column blocks are the outer loop, so consecutive tiles walk the groups of one column
band: a window shared by consecutive groups of one expert stays where it was fetched.
"""

import tilejax_amd as autokernel
from tilejax_amd.jaxlite import jax, jnp


@autokernel.tunable
class GroupTiles:
    """Output columns per tile, and the reduction depth per step (the rows per tile are the group size)."""

    tn: int = autokernel.choice(256, 512, 1024, 2048, default=512)
    tk: int = autokernel.choice(256, 512, 1024, 2048, 4096, default=512)


@autokernel.kernel
def grouped_matmul(xs, w, group_expert, tiles=GroupTiles()):
    M, K = xs.shape
    E, _, N = w.shape
    G = M // group_expert.shape[0]
    tn, tk = min(tiles.tn, N), min(tiles.tk, K)
    dtype = xs.dtype
    out = jnp.zeros((M, N), dtype)
    for j in range(0, N, tn):
        for i in range(0, M, G):
            acc = jnp.zeros((G, tn), jnp.float32)
            for k in range(0, K, tk):
                if group_expert[i // G] < 0:  # an unused group: decided on the device, before the kernel runs
                    continue
                acc += xs[i : i + G, k : k + tk] @ w[group_expert[i // G], k : k + tk, j : j + tn]
            out = out.at[i : i + G, j : j + tn].set(acc.astype(dtype))
    return out


@autokernel.tunable
class ExpertTiles:
    """Hidden units of an expert per step (the rows per tile are the layout's group size)."""

    block_f: int = autokernel.choice(128, 256, 512, 1024, 2048, default=256)


@autokernel.kernel
def expert_ffn(xs, w_gate, w_up, w_down, tile_expert, tiles=ExpertTiles()):
    """The reference's runtime-window MoE layer (examples/moe.py:167-187): each tile of G rows of `xs` through
    its expert's SwiGLU feed-forward layer, `tile_expert[t]` naming tile t's expert (-1 for an unused tile,
    whose rows stay zero). Three products per step, a SiLU between them: no matmul-family shape, so it lowers
    to the generic kernel (with device-built step tables for its runtime mask)."""
    M, D = xs.shape
    F = w_gate.shape[2]
    G = M // tile_expert.shape[0]
    bf = min(tiles.block_f, F)
    dtype = xs.dtype
    out = jnp.zeros((M, D), dtype)
    for i in range(0, M, G):
        acc = jnp.zeros((G, D), jnp.float32)
        for f in range(0, F, bf):  # the expert's hidden units, bf per step
            if tile_expert[i // G] < 0:  # an unused tile: decided on the device
                continue
            xt = xs[i : i + G, :]
            g = xt @ w_gate[tile_expert[i // G], :, f : f + bf]
            u = xt @ w_up[tile_expert[i // G], :, f : f + bf]
            acc += (jax.nn.silu(g) * u).astype(dtype) @ w_down[tile_expert[i // G], f : f + bf, :]
        out = out.at[i : i + G, :].set(acc.astype(dtype))
    return out
