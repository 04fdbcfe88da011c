"""Load the reference-side binding module that INTEGRATION.md shows (its
``apexw/rocm_extension.py`` code block), so tests run exactly that code."""

import os
import re
import types

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def load_binding():
    from apexw_amd import _lib
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    m = re.search(r"## Reference-side binding[^\n]*\n+```python\n(.*?)\n```", text, re.S)
    assert m, "INTEGRATION.md has no reference-side binding block"
    os.environ["APEXW_HIP_LIB"] = _lib.LIB_PATH
    mod = types.ModuleType("rocm_extension")
    exec(compile(m.group(1), "INTEGRATION.md:rocm_extension", "exec"), mod.__dict__)
    return mod
