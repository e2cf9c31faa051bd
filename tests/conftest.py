import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for sub in ("", "metal-infer-rs_amd", "oracle", "tests"):
    path = str(ROOT / sub) if sub else str(ROOT)
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libmi_attn.so)")


@pytest.fixture(scope="session")
def ctx():
    """One HIP context for the whole GPU session (fails loudly without a GPU)."""
    import mi_attn

    context = mi_attn.Context(0)
    print(f"[ctx] {context.device_name}, {context.compute_units} CUs", flush=True)
    yield context
    context.close()
