"""The C-ABI library loads and exports every entry point include/esp_hip.h
declares (no compute calls: this runs without a GPU)."""
import ctypes
import os
import re

from esp_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(ROOT, "include", "esp_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"typedef[^;]*\(\s*\*[^;]*;", "", text)  # function-pointer types
    return sorted(set(re.findall(r"\b(esp_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared()
    assert len(names) >= 17
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(_lib.EXPORTED) == names


def test_version_and_error_buffer_without_gpu():
    lib = _lib.load()
    assert b"gfx950" in lib.esp_version()
    buf = ctypes.create_string_buffer(8)
    n = lib.esp_last_error(buf, 8)
    assert n == len(buf.value)


def test_struct_layouts_match_header():
    # esp_config: 19 u32/f32 scalars, a pointer, 5 u32, a pointer, 1 u32
    assert ctypes.sizeof(_lib.EspSampler) == 16
    assert ctypes.sizeof(_lib.EspLora) == 32
    assert _lib.EspConfig.format.offset > _lib.EspConfig.layer_is_moe.offset
