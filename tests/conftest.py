import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; parity tests through the C-ABI")


def _gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible (gpu tests run on the MI355X box)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    oracle.build()
    return oracle


@pytest.fixture(scope="session")
def dispatch_via_reference_loader(tmp_path_factory):
    """The built pdscope_layer_dispatch extension, loaded the way the
    reference driver loads its native module (benchmarks/pdscope_compare.py:
    39-52): the first match of the glob
    expertbench/native-build/layer-dispatch/pdscope_layer_dispatch*.so under
    the tree's root, then spec_from_file_location / module_from_spec /
    exec_module, then the submit_and_merge check.  The file is placed there
    as a symlink to the package's build, which is how a user of the
    reference installs it."""
    import importlib.util
    from pdscope_amd import build as B
    root = tmp_path_factory.mktemp("reference_tree")
    where = root / "expertbench" / "native-build" / "layer-dispatch"
    where.mkdir(parents=True)
    (where / B.DISPATCH_MODULE.name).symlink_to(B.DISPATCH_MODULE)
    candidates = sorted(where.glob("pdscope_layer_dispatch*.so"))
    assert candidates, "native layer dispatch is not built"
    spec = importlib.util.spec_from_file_location("pdscope_layer_dispatch", candidates[0])
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    assert hasattr(module, "submit_and_merge"), "native dispatch lacks submit_and_merge"
    return module
