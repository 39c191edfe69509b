"""The C-ABI library loads on a CPU-only machine and exports every symbol include/kvq.h declares,
with the ctypes signatures the Python side binds (no compute call: that needs a GPU)."""
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _declared():
    text = (ROOT / "include" / "kvq.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kvq_[a-z0-9_]+)\s*\(", text)))


def _ensure_built():
    from kvq import _lib
    if not _lib.LIB_PATH.exists():
        import kvq.build as b
        b.build()
    return _lib


def test_library_exports_every_declared_symbol():
    _lib = _ensure_built()
    lib = _lib.load()
    names = _declared()
    assert names, "no declarations parsed"
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/kvq.h but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert lib.kvq_abi_version() == 18
    assert lib.kvq_last_error() == b""


def test_argument_validation_without_gpu():
    # rejected before any launch: no device needed
    _lib = _ensure_built()
    lib = _lib.load()
    rc = lib.kvq_pack_codes(None, 10, 3, None, None)
    assert rc == 1 and b"bits" in lib.kvq_last_error()
    rc = lib.kvq_kivi_decode(None, 0, 0, 0, 0, 1, 8, 8, 1, 64, 0.1, None, None, None, None, None, 64, 0, 32, 32,
                             None, None, 0, 1, 1, None, None, None, 0, None, 0, None, 0, 0.0, 0, 3, None)
    assert rc == 1 and b"head_dim" in lib.kvq_last_error()
    assert lib.kvq_kivi_decode_workspace(16, 32, 8, 1, 128, 32640, 128, 64, 64, 0) > 0


def test_split_plan_fills_one_round():
    """Automatic split (16x8 (b, h), 32640 packed + 128 exact tokens, 3 resident blocks per CU on
    256 CUs): 6 packed splits per (b, h) = 768 blocks, one round, so the plan is class-major and the
    128 window rows go to 2 exact-row blocks of 64 rows per (b, h) in the same launch.  Off that
    one-round shape, exact windows of at most 1024 rows are attended by the merge (no exact-row
    blocks, no partials); longer ones are blocks of 64 rows dispatched after the packed blocks.  The
    workspace holds S1 * rows * (d + 2) + 2 * rows floats per (b, h), S1 = exact-row blocks + packed
    splits (partials, then each row's max and sum)."""
    from kvq import _lib
    lib = _lib.load()
    BH, R, d = 16 * 8, 4, 128
    assert lib.kvq_kivi_decode_workspace(16, 32, 8, 1, 128, 32640, 128, 64, 64, 0) == BH * (8 * R * (d + 2) + 2 * R)
    assert lib.kvq_kivi_decode_workspace(16, 32, 8, 1, 128, 32640, 0, 64, 64, 0) == BH * (6 * R * (d + 2) + 2 * R)
    # explicit split size: ceil(n_q / split_tokens) splits
    assert lib.kvq_kivi_decode_workspace(16, 32, 8, 1, 128, 32640, 128, 64, 64, 3000) == BH * (11 * R * (d + 2) + 2 * R)
    assert lib.kvq_kivi_decode_workspace(16, 32, 8, 1, 128, 32640, 128, 64, 48, 0) == -1
    # exact rows only (in the merge / in blocks of 64) / packed rows only
    assert lib.kvq_kivi_decode_workspace(1, 8, 8, 1, 128, 0, 100, 32, 32, 0) == 8 * (0 * 1 * (d + 2) + 2)
    assert lib.kvq_kivi_decode_workspace(1, 8, 8, 1, 128, 0, 2304, 32, 32, 0) == 8 * (36 * 1 * (d + 2) + 2)
    assert lib.kvq_kivi_decode_workspace(1, 8, 8, 1, 128, 64, 0, 32, 32, 0) == 8 * (1 * 1 * (d + 2) + 2)


def test_noalloc_rejects_steps_beyond_the_static_scratch():
    """kvq_kivi_decode_noalloc refuses, before touching the device, a step whose partials exceed its
    static scratch (KVQ_NOALLOC_SCRATCH_FLOATS = 2^21 floats); C2 itself fits (400,384)."""
    from kvq import _lib
    lib = _lib.load()
    assert lib.kvq_kivi_decode_workspace(16, 32, 8, 1, 128, 32640, 128, 64, 64, 0) <= 1 << 21
    assert lib.kvq_kivi_decode_workspace(512, 32, 8, 1, 128, 32640, 128, 64, 64, 0) > 1 << 21
    rc = lib.kvq_kivi_decode_noalloc(None, 2, 0, 0, 0, 512, 32, 8, 1, 128, 0.1, None, None, None, None, None,
                                     32640, 32640, 64, 64, None, None, 2, 128, 128, None, None, None, 2, None, 0,
                                     0.0, 0, 3, None)
    assert rc == 1 and b"static scratch" in lib.kvq_last_error()
