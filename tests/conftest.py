"""Shared pytest setup: import paths and the `gpu` marker.

GPU tests run on a machine with a HIP device. Where no GPU exists at all
(no /dev/kfd) they are skipped; on a machine that has /dev/kfd but where torch
cannot see the GPU they fail, so a broken GPU setup is never a silent pass.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "inference-speech-model_amd")
for p in (PKG, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

import pytest  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X)")


_LIBRARY_STATE = {}


def _library_is_current():
    """Build libspeechkv.so when none is built (a host without ROCm skips the tests that need it);
    fail every such test when the built one does not come from the sources in this tree (a stale
    binary must never pass the GPU suite). Checked once, for the tests that load the library."""
    if "outcome" not in _LIBRARY_STATE:
        from speech_serving import native

        outcome = ("ok", "")
        if not os.path.exists(native.library_path()):
            import build  # inference-speech-model_amd/build.py

            try:
                build.build()
            except RuntimeError as e:
                outcome = ("skip", f"libspeechkv.so is not built and cannot be built here: {e}")
        if outcome[0] == "ok":
            try:
                native.lib()
            except RuntimeError as e:
                outcome = ("fail", f"libspeechkv.so does not match the checked-out sources: {e}")
        _LIBRARY_STATE["outcome"] = outcome
    kind, msg = _LIBRARY_STATE["outcome"]
    if kind == "skip":
        pytest.skip(msg)
    if kind == "fail":
        pytest.fail(msg, pytrace=False)


@pytest.fixture(autouse=True)
def _speechkv_library(request):
    """The GPU tests and the C-ABI tests run against a library built from this tree."""
    if "gpu" in request.keywords or request.node.nodeid.replace(os.sep, "/").split("::")[0].endswith("test_abi.py"):
        _library_is_current()


def pytest_collection_modifyitems(config, items):
    if os.path.exists("/dev/kfd"):
        return
    skip = pytest.mark.skip(reason="no GPU on this machine (/dev/kfd absent)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test on a machine with /dev/kfd but torch.cuda.is_available() is False")
    return torch.device("cuda", 0)
