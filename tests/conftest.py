import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def load_package():
    """Import the package directory omlx-exl3_amd/ under the module name omlx_exl3_amd."""
    name = "omlx_exl3_amd"
    if name in sys.modules:
        return sys.modules[name]
    pkg_dir = os.path.join(ROOT, "omlx-exl3_amd")
    spec = importlib.util.spec_from_file_location(name, os.path.join(pkg_dir, "__init__.py"),
                                                  submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built HIP library")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if gpu_available():
        return
    skip = pytest.mark.skip(reason="no HIP device in this container")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


class LibCalls:
    """Counts the C-ABI kernel entry points the package calls while the context is active, by wrapping the
    loaded library handle (queries such as exl3_last_error and exl3_gemv_workspace_bytes are not counted)."""

    QUERIES = ("exl3_last_error", "exl3_gemv_workspace_bytes", "exl3_version")

    def __init__(self):
        import collections
        self.counts = collections.Counter()

    def __enter__(self):
        from omlx_exl3_amd import _capi
        real = _capi.lib()
        counts = self.counts

        class _Proxy:
            def __getattr__(self, name):
                fn = getattr(real, name)
                if not name.startswith("exl3_") or name in LibCalls.QUERIES:
                    return fn

                def call(*args):
                    counts[name] += 1
                    return fn(*args)
                return call

        self._capi, self._real = _capi, real
        _capi._lib = _Proxy()
        return self

    def __exit__(self, *exc):
        self._capi._lib = self._real
        return False

    def total(self) -> int:
        return sum(self.counts.values())
