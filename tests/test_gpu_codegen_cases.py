"""The loop nests of tests/codegen_cases.py on the GPU, each kernel against its float64 closed form."""

import pytest
import torch

from tests.codegen_cases import CASES, check
from tests.helpers import make_kernel

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", CASES, ids=lambda c: c.name)
def test_kernel(case):
    kernel = make_kernel(case.source, **case.namespace)
    inputs = case.inputs()
    lowered = kernel.lower(*inputs)
    print(f"codegen case: {case.name} -> {lowered.program.notes['family']} "
          f"{[tuple(t.shape) for t in inputs]}", flush=True)
    got = lowered.run(*(t.cuda() for t in inputs))
    torch.cuda.synchronize()
    got = tuple(g.cpu() for g in got) if isinstance(got, tuple) else got.cpu()
    check(case, got, case.want(*inputs))
