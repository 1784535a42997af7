"""The binding stubs INTEGRATION.md shows a maintainer of the reference are valid Python."""

import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_integration_python_blocks_compile():
    text = (ROOT / "INTEGRATION.md").read_text()
    blocks = re.findall(r"```python\n(.*?)```", text, re.S)
    assert blocks, "INTEGRATION.md shows no Python bindings"
    for i, code in enumerate(blocks):
        compile(code, f"INTEGRATION.md python block {i}", "exec")
