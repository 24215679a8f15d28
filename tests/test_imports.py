"""Every relative import in the package names a module and attribute that exist (imports inside functions
included, which only run on the GPU paths)."""

import importlib
import os
import re

ROOT = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "tilejax_amd")


def test_relative_imports_resolve():
    missing = []
    for here, _, files in os.walk(ROOT):
        package = os.path.relpath(here, os.path.dirname(ROOT)).replace(os.sep, ".")
        for f in files:
            if not f.endswith(".py"):
                continue
            text = open(os.path.join(here, f)).read()
            for dots, mod, names in re.findall(r"from (\.+)(\w*) import ([\w, ]+(?: as \w+)?)", text):
                parts = package.split(".")
                parts = parts[: len(parts) - (len(dots) - 1)] + ([mod] if mod else [])
                module = importlib.import_module(".".join(parts))
                for name in (n.strip().split(" as ")[0] for n in names.split(",")):
                    if name and not hasattr(module, name):
                        try:
                            importlib.import_module(f"{module.__name__}.{name}")
                        except ImportError:
                            missing.append(f"{f}: {module.__name__}.{name}")
    assert not missing, missing
