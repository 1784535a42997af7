"""The Python binding stubs of the integration guide (the file read below) compile."""

import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_integration_python_blocks_compile():
    text = (ROOT / "INTEGRATION.md").read_text()
    blocks = re.findall(r"```python\n(.*?)```", text, re.S)
    assert blocks, "the integration guide shows no Python bindings"
    for i, code in enumerate(blocks):
        compile(code, f"INTEGRATION.md python block {i}", "exec")


def test_integration_stub_argtypes_match_the_library_bindings():
    # every `lib.<entry>.argtypes = [...]` the guide shows has the argument
    # types the package's own binding declares for that entry point
    import ctypes

    from kotodama_amd import _capi

    text = (ROOT / "INTEGRATION.md").read_text()
    code = "\n".join(re.findall(r"```python\n(.*?)```", text, re.S))
    ns = {"ctypes": ctypes, "vp": ctypes.c_void_p, "i64": ctypes.c_int64, "i32": ctypes.c_int, "f32": ctypes.c_float}
    stubs = re.findall(r"lib\.(attnres_\w+)\.argtypes = (\[.*?\])", code, re.S)
    assert stubs, "the integration guide shows no argtypes"
    for name, rhs in stubs:
        shown = eval(rhs, ns)  # noqa: S307 - a list of ctypes types from the repository's own guide
        declared = _capi._SIGNATURES[name][0]
        assert shown == list(declared), f"{name}: the guide's argtypes differ from the binding's"
