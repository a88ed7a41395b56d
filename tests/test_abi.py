"""The C-ABI boundary without a GPU: the library loads, exports every function
include/leo_hip.h declares, the generated config layout matches leo_abi.def,
and an explicit GPU request fails loudly instead of falling back to the CPU
(docs/ADR-0001-EXECUTION-BACKENDS.md:9)."""
from __future__ import annotations

import ctypes
import pathlib
import re
import subprocess
import sys

import pytest

from leo_amd import _abi, native
from leo_amd.model import Model, host_config
from tests.helpers import toml_test_config

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _declared_functions(header="leo_hip.h"):
    text = (ROOT / "include" / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"^\s*(?:[A-Za-z_][\w\s\*]*?)\b(leo_\w+)\s*\(", text, flags=re.M))


def test_header_declares_the_backend_surface():
    names = _declared_functions()
    for required in ("leo_hip_create", "leo_hip_destroy", "leo_hip_step", "leo_hip_training_step_batch",
                     "leo_hip_advance_frozen_batch", "leo_hip_training_story_batch", "leo_hip_train_batch",
                     "leo_hip_download_model", "leo_hip_upload_model", "leo_hip_parameter_changes",
                     "leo_hip_last_error"):
        assert required in names


def test_library_exports_every_declared_function():
    lib = ctypes.CDLL(str(native.LIB_PATH))
    declared = _declared_functions() | _declared_functions("leo_formats.h")
    missing = [name for name in sorted(declared) if not hasattr(lib, name)]
    assert not missing, f"declared but not exported: {missing}"


def test_python_signatures_cover_exactly_the_header():
    assert set(native.SIGNATURES) == _declared_functions()
    assert set(native.FORMAT_SIGNATURES) == _declared_functions("leo_formats.h")


def test_generated_abi_is_current():
    subprocess.run([sys.executable, str(ROOT / "leo_amd" / "csrc" / "gen_abi.py"), "--check"], check=True)


def test_device_config_layout_matches_the_reference_abi():
    # 14 u32 then 26 f32 (crates/leo-core/src/cuda_abi.def:5-44)
    assert ctypes.sizeof(_abi.LeoConfig) == 160
    kinds = [t for _, t in _abi.LeoConfig._fields_]
    assert kinds[:14] == [ctypes.c_uint32] * 14 and kinds[14:] == [ctypes.c_float] * 26
    assert _abi.LeoConfig._fields_[0][0] == "neuron_count"


def test_abi_version():
    assert native.load().leo_hip_abi_version() == 1


def test_gpu_request_without_a_device_fails_loudly():
    if _gpu_present():
        pytest.skip("a HIP device is present")
    model = Model.initialize(toml_test_config())
    from leo_amd.runtime import HipRuntime

    with pytest.raises(native.LeoError) as err:
        HipRuntime(model, device=0, max_lanes=1)
    assert err.value.code == native.ERR_DEVICE


def test_null_arguments_are_rejected():
    lib = native.load()
    assert lib.leo_hip_create(None, None, 0, 1, None) == native.ERR_INVALID_ARGUMENT
    assert "null" in native.last_error(lib)
    assert lib.leo_hip_step(None, 0, -1, native.TRAINING, None) == native.ERR_INVALID_ARGUMENT


def test_invalid_model_is_rejected_before_the_device():
    cfg = toml_test_config()
    model = Model.initialize(cfg)
    model.threshold[0] = float("nan")
    lib = native.load()
    hc = host_config(cfg)
    view = model.view()
    handle = ctypes.c_void_p()
    status = lib.leo_hip_create(ctypes.byref(hc), ctypes.byref(view), 0, 1, ctypes.byref(handle))
    assert status == native.ERR_INVALID_ARGUMENT, native.last_error(lib)


def _gpu_present() -> bool:
    from tests.conftest import gpu_available

    return gpu_available()
