import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def plans(tmp_path_factory):
    """Random-init plans written once per session: name -> (plan path, FLOPs/image)."""
    from infvino_amd import planwriter as pw
    base = tmp_path_factory.mktemp("plans")
    cache = {}

    def get(name, **kw):
        key = (name, tuple(sorted(kw.items())))
        if key not in cache:
            d = str(base / (name + "_" + "_".join(f"{k}{v}" for k, v in sorted(kw.items()))))
            if name in pw.MODELS:
                cache[key] = pw.MODELS[name](d, **kw)
            else:
                cache[key] = getattr(pw, name)(d, **kw)
        return cache[key]
    return get
