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
