"""CPU tests of the C-ABI boundary: the library loads, exports every entry
point include/*.h declares, and rejects bad arguments with a status instead
of crashing (no device work is done here)."""
import ctypes as C
import os
import re

import pytest

import qtts

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in ("qtts.h", "qtts_synth.h", "qtts_file.h", "qtts_decoder.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(qtts_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_every_declared_symbol_is_exported():
    lib = qtts.load_library()
    decl = declared_symbols()
    assert len(decl) >= 35
    for name in decl:
        assert hasattr(lib, name), name
    assert sorted(qtts.exported_symbols()) == decl


def test_version_string():
    assert b"gfx950" in qtts.load_library().qtts_version()


def test_null_arguments_are_rejected():
    lib = qtts.load_library()
    assert lib.qtts_ctx_create(0, None) == qtts.QTTS_EINVAL
    assert lib.qtts_gemv(None, None, None, None) == qtts.QTTS_EINVAL
    assert lib.qtts_forward_with_embedding(None, None, None, 0, None) == qtts.QTTS_EINVAL
    assert lib.qtts_sample_token(None, None, 0, None, None, 0, None, None) == qtts.QTTS_EINVAL
    assert lib.qtts_kv_len(None) == -1
    assert lib.qtts_prefill_talker(None, None, None, 1, None, None) == qtts.QTTS_EINVAL
    assert lib.qtts_generate_speech(None, None, None, None, 0, 0, 0, None, None, None, None, 0, None, 0, None,
                                    None) == qtts.QTTS_EINVAL
    # the read-floor aid refuses a null buffer, a size off the 16-byte grid
    # and an unaligned buffer before any device work
    assert lib.qtts_stream_read_device(None, 16, None) == -1
    assert lib.qtts_stream_read_device(C.c_void_p(4096), 24, None) == -1
    assert lib.qtts_stream_read_device(C.c_void_p(4100), 32, None) == -1
    assert lib.qtts_stream_read_device_ex(None, 16, 0, 1, None) == -1
    assert lib.qtts_stream_read_device_ex(C.c_void_p(4096), 32, 8, 3, None) == -1
    assert lib.qtts_stream_read_device_ex(C.c_void_p(4096), 32, -1, 4, None) == -1
    assert lib.qtts_last_error(None) == b"null context"
    lib.qtts_ctx_destroy(None)
    lib.qtts_q4_free(None)
    lib.qtts_kv_free(None)


def _has_gpu():
    try:
        import torch  # noqa: F401  (device count only; does not initialise HIP)

        return torch.cuda.device_count() > 0
    except Exception:
        return False


@pytest.mark.skipif(_has_gpu(), reason="checks the no-device path")
def test_context_without_device_reports_edevice():
    h = C.c_void_p()
    assert qtts.load_library().qtts_ctx_create(0, C.byref(h)) == qtts.QTTS_EDEVICE
    assert not h.value
