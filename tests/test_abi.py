"""CPU tests of the C ABI: the library loads, exports every symbol the header
declares, and its host-side planner reproduces the reference dispatcher's
routing and split plan (checked against the oracle).  No GPU is touched."""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

import oracle
from inferno_amd import _lib
from inferno_amd.kv import FULL, SLIDING, AttentionPlan, KVRunTable
from tests.helpers import KV_STRIDE, PAGE_LEN, make_decode_case, make_prefill_case

INCLUDE = Path(__file__).resolve().parent.parent / "include"
HEADERS = [INCLUDE / "inferno_hip.h", INCLUDE / "inferno_host.h"]


def declared_functions():
    names = set()
    for h in HEADERS:
        names.update(re.findall(
            r"^(?:int32_t|int64_t|uint64_t|void|ifr_\w+\s*\*)\s*(ifr_\w+)\s*\(",
            h.read_text(), re.M))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_functions()
    assert len(names) >= 75
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(_lib.SIGNATURES) == names
    assert lib.ifr_abi_version() == 1


def test_partial_stride_matches_reference():
    assert _lib.lib().ifr_flash_partial_stride(16, 256) == oracle.flash_partial_stride(16, 256)


def _plan(table_runs, rows, seq_len, kind, window, cache_size, cache_rows, cap, row_bytes):
    lib = _lib.lib()
    runs = np.ascontiguousarray(table_runs, dtype=np.int32)
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    nbytes = lib.ifr_plan_bytes(runs.shape[0], rows.shape[0], seq_len, cap)
    img = np.zeros(nbytes // 4, dtype=np.int32)
    info = (C.c_int64 * 16)()
    st = lib.ifr_plan_attention(img.ctypes.data, img.nbytes,
                                runs.ctypes.data_as(_lib.P_I32), runs.shape[0],
                                rows.ctypes.data_as(_lib.P_I32), rows.shape[0], seq_len,
                                kind, window, cache_size, PAGE_LEN, cache_rows, cap,
                                row_bytes, info)
    return st, img, list(info)


def _items(img, info):
    off, n = img[11], info[0]
    return img[off:off + 8 * n].reshape(n, 8)[:, :6]


def _units(img, info):
    off, n = img[12], info[1]
    return img[off:off + 4 * n].reshape(n, 4)[:, :3]


@pytest.mark.parametrize("cap", [1, 7, 64, 65, 256, 2048])
def test_batched_plan_matches_oracle(cap):
    rng = np.random.default_rng(cap)
    ctx = [int(x) for x in rng.integers(512, 32768, 64)]
    case = make_decode_case(cap, ctx)
    st, img, info = _plan(case.runs, case.base_rows, 64, FULL, 0, PAGE_LEN,
                          case.cache_rows, cap, KV_STRIDE * 2)
    assert st == 0, _lib.last_error()
    items, units = _items(img, info), _units(img, info)
    kv = [c + 1 for c in ctx]
    if 64 < cap:
        assert info[2] == _lib.PLAN_SPLIT_MERGE
        bands = oracle.plan_run_splits(kv, list(range(64)), cap, 16)
        assert np.array_equal(units[:, 1], bands[:, 1])
        assert np.array_equal(units[:, 2], bands[:, 2])
        expect = []
        for i in range(64):
            for s in range(bands[i, 2]):
                a, b = oracle.worker_range(kv[i], int(bands[i, 2]), s)
                expect.append([i, i, 0, a, b, int(bands[i, 1]) + s])
        # Items are dispatched longest first (a stable sort on end - start);
        # each names its own stripe, so the order changes no result.
        expect.sort(key=lambda r: -(r[4] - r[3]))
        assert [list(map(int, r)) for r in items] == expect
        assert info[3] == bands[:, 2].sum() == min(cap, sum((x + 15) // 16 for x in kv))
    else:  # token-partitioned route: one item per token over its whole range
        assert info[2] == _lib.PLAN_TOKEN_MERGE
        assert [list(r) for r in items] == [[i, i, 0, 0, kv[i], i] for i in range(64)]


def test_single_token_plan_uses_recommended_workers():
    case = make_decode_case(1, [4096])
    for cap, kind in [(128, FULL), (3, FULL), (96, SLIDING)]:
        window = 1024
        cache_size = 128 * PAGE_LEN if kind == SLIDING else PAGE_LEN
        runs = case.runs.copy()
        rows = case.base_rows
        if kind == SLIDING:
            runs[0, 3] = 128
            rows = np.concatenate([rows, np.zeros(128 - rows.size, dtype=np.int32)])
        st, img, info = _plan(runs, rows, 1, kind, window, cache_size, case.cache_rows,
                              cap, KV_STRIDE * 2)
        assert st == 0, _lib.last_error()
        valid = 4097 if kind == FULL else 1024
        nw = min(oracle.recommended_workers(valid * KV_STRIDE * 2, cap), cap, valid)
        items = _items(img, info)
        start_pos = 0 if kind == FULL else 4096 - 1024 + 1
        assert [tuple(r) for r in items] == [
            (0, 0, start_pos) + oracle.worker_range(valid, nw, w) + (w,) for w in range(nw)]


def test_prefill_plan_and_token_map():
    case = make_prefill_case(2, [0, 130, 64], [40, 7, 64])
    n = 40 + 7 + 64
    st, img, info = _plan(case.runs, case.base_rows, n, FULL, 0, PAGE_LEN,
                          case.cache_rows, 16, KV_STRIDE * 2)
    assert st == 0, _lib.last_error()
    assert info[2] == _lib.PLAN_TOKEN_MERGE and info[0] == n
    tokrun = img[img[10]:img[10] + n]
    assert list(tokrun) == [0] * 40 + [1] * 7 + [2] * 64
    items = _items(img, info)
    assert list(items[45]) == [45, 1, 0, 0, 130 + 5 + 1, 45]


def test_planner_rejects_out_of_cache_pages():
    case = make_decode_case(3, [100, 200])
    st, _, _ = _plan(case.runs, case.base_rows, 2, FULL, 0, PAGE_LEN,
                     case.cache_rows - 1, 16, KV_STRIDE * 2)
    assert st == _lib.lib().ifr_abi_version() * 0 - 1 and "outside cache" in _lib.last_error()
    runs = case.runs.copy()
    runs[1, 3] = 1  # too few pages for position 200
    st, _, _ = _plan(runs, case.base_rows, 2, FULL, 0, PAGE_LEN, case.cache_rows, 16,
                     KV_STRIDE * 2)
    assert st == -1 and "needs" in _lib.last_error()
    st, _, _ = _plan(case.runs, case.base_rows, 2, SLIDING, 64, 3 * PAGE_LEN,
                     case.cache_rows, 16, KV_STRIDE * 2)
    assert st == -1  # ring of 3 pages is not a power of two


def test_plan_image_too_small_is_reported():
    lib = _lib.lib()
    case = make_decode_case(4, [10])
    info = (C.c_int64 * 16)()
    img = np.zeros(4, dtype=np.int32)
    st = lib.ifr_plan_attention(img.ctypes.data, img.nbytes,
                                case.runs.ctypes.data_as(_lib.P_I32), 1,
                                case.base_rows.ctypes.data_as(_lib.P_I32), 1, 1, FULL, 0,
                                PAGE_LEN, PAGE_LEN, case.cache_rows, 4, 4096, info)
    assert st == -4


@pytest.mark.parametrize("layout", ["empty_first_single", "empty_middle_batched"])
def test_planner_rejects_runs_without_tokens(layout):
    """A run with no token would be planned over rows of no token of the
    step (seq_len 1 plans run 0; the batched route plans one run per token):
    the planner refuses it instead of letting the kernels read those rows."""
    case = make_decode_case(6, [300, 700, 90])
    runs = case.runs.copy()
    if layout == "empty_first_single":
        # Run 0 empty, run 1 holds the step's one token.
        runs = runs[:2].copy()
        runs[:, 0] = [0, 0]
        seq_len = 1
    else:
        # Three runs over two tokens: run 1 is empty.
        runs[:, 0] = [0, 1, 1]
        seq_len = 2
    st, _, _ = _plan(runs, case.base_rows, seq_len, FULL, 0, PAGE_LEN, case.cache_rows, 16,
                     KV_STRIDE * 2)
    assert st == -1 and "no token" in _lib.last_error()


def _header_prototypes():
    """name -> (return C type, [param C types]) from both headers."""
    protos = {}
    for h in HEADERS:
        src = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"^\s*([a-z_0-9]+(?:\s*\*)?)\s+(ifr_\w+)\s*\(([^;]*?)\)\s*;", src,
                             re.M | re.S):
            params = [" ".join(a.split()) for a in m.group(3).split(",")]
            params = [re.match(r"(.*?)\w+$", a).group(1).strip() for a in params
                      if a not in ("void", "")]
            protos[m.group(2)] = (m.group(1).strip(), params)
    return protos


def test_mojo_bindings_match_headers():
    """include/inferno_hip.mojo has one wrapper per declared C function, with
    the same arity, the agreed type mapping (pointers as Int64 addresses,
    int64_t Int64, uint64_t UInt64, int32_t Int32, float Float32), and each
    wrapper calls its own symbol with its parameters in order."""
    def mojo_type(c):
        c = c.replace("const ", "").strip()
        if c.endswith("*"):
            return "Int64"
        return {"int64_t": "Int64", "uint64_t": "UInt64", "int32_t": "Int32",
                "float": "Float32"}[c]

    protos = _header_prototypes()
    text = (INCLUDE / "inferno_hip.mojo").read_text()
    defs = re.findall(r"^def (ifr_\w+)\((.*?)\)(?: -> (\w+))?:\n(.*?)(?=\n\n|\Z)", text,
                      re.M | re.S)
    assert sorted(d[0] for d in defs) == sorted(protos), "wrapper set differs from the headers"
    for name, params, ret, body in defs:
        cret, cparams = protos[name]
        ps = [p.strip() for p in params.split(",") if p.strip()]
        names = [p.split(":")[0].strip() for p in ps]
        types = [p.split(":")[1].strip() for p in ps]
        assert types == [mojo_type(c) for c in cparams], name
        want_ret = None if cret == "void" else mojo_type(cret)
        assert (ret or None) == want_ret, name
        assert f'func = "{name}".value' in body, name
        call = re.search(r"\]\((.*?)\)\s*$", body, re.S).group(1)
        assert [a.strip() for a in call.split(",") if a.strip()] == names, name
