"""The loop nests of tests/codegen_cases.py on the CPU: `kernel.reference` (the nest run eagerly) against
each float64 closed form, and the kernel each lowers to builds for gfx950 (its family named)."""

import pytest

from tests.codegen_cases import CASES, check
from tests.helpers import make_kernel
from tilejax_amd import runtime


@pytest.mark.parametrize("case", CASES, ids=lambda c: c.name)
def test_reference_and_kernel_build(case):
    kernel = make_kernel(case.source, **case.namespace)
    inputs = case.inputs()
    check(case, kernel.reference(*inputs), case.want(*inputs))
    lowered = kernel.lower(*inputs)
    print(f"  {case.name}: {lowered.program.notes['family']}", flush=True)
    runtime.compile_source(lowered.source, f"{lowered.program.name}.hip")
