"""Bounded fuzz of the safetensors header parser behind astro_moe_safetensors_tensor (CPU).

Every case is a seeded mutation of a valid file: bytes flipped, JSON tokens inserted or
deleted, spans duplicated or swapped, number literals swapped for edge values, the length
prefix moved.  The library's verdict on each case is compared with `model_parse`, a
restatement here of the reference's header reading:
  - framing and the 64 MiB limit: safetensors/header.rs:109-158;
  - the JSON it accepts (serde_json 1.0.151 `from_slice` through the duplicate-rejecting value
    of strict_json.rs:11-110): strict UTF-8, finite numbers, "-0" read as a float, integers
    as i64 only where they fit, at most 127 nested containers (serde_json's recursion limit);
  - the entry checks in key order (serde_json's map is ordered by key):
    expert_paging/safetensors_header.rs:171-276 and :358-430.
The model uses Python's json module as the JSON reader, so the C parser is checked against an
independent reader, not against a copy of itself.  A case passes when both reject it with the
same error class (and the same tensor, where the message names one), or both accept it with
identical entries for every tensor.  The library must never crash or hang on a case:
tests/sanitize/run.sh runs this file against the AddressSanitizer + UBSan build of the parser.
"""
import json
import math
import os
import random
import time

import pytest

from astronomical_amd import pages as P
from astronomical_amd._lib import AstroMoeError, INVALID_ARGUMENT

MAX_HEADER = 64 << 20
MAX_NESTING = 127
WIDTHS = {"BOOL": 1, "I8": 1, "U8": 1, "F8_E4M3": 1, "F8_E5M2": 1, "I16": 2, "U16": 2, "F16": 2,
          "BF16": 2, "I32": 4, "U32": 4, "F32": 4, "I64": 8, "U64": 8}
I64 = (-(1 << 63), 1 << 63)


class _Reject(Exception):
    pass


def _pairs(pairs):
    d = {}
    for k, v in pairs:
        if k in d:
            raise _Reject("duplicate key")
        d[k] = v
    return d


def _int(s):
    if s == "-0":
        return -0.0  # serde_json: a float
    try:
        v = int(s)
    except ValueError:  # beyond Python's digit limit: far beyond f64 as well
        raise _Reject("number out of range")
    if -(1 << 63) <= v < (1 << 64):
        return v
    f = float(s)
    if math.isinf(f):
        raise _Reject("number out of range")
    return f


def _float(s):
    f = float(s)
    if math.isinf(f):
        raise _Reject("number out of range")
    return f


def _const(s):
    raise _Reject("not JSON: " + s)


def _check_tree(v, depth=0):
    """Lone surrogates and nesting beyond the limit (containers nested in containers)."""
    if isinstance(v, str):
        if any(0xD800 <= ord(c) <= 0xDFFF for c in v):
            raise _Reject("lone surrogate")
    elif isinstance(v, (list, dict)):
        if depth >= MAX_NESTING:
            raise _Reject("nesting")
        items = v.items() if isinstance(v, dict) else enumerate(v)
        for k, x in items:
            if isinstance(k, str):
                _check_tree(k, depth + 1)
            _check_tree(x, depth + 1)


def _is_i64(v):
    return isinstance(v, int) and not isinstance(v, bool) and I64[0] <= v < I64[1]


def model_parse(data: bytes):
    """('ok', {name: (dtype, shape, start, end)}) or ('err', error class, tensor name or None)."""
    if len(data) < 8:
        return ("err", "too small to contain a header length prefix", None)
    n = int.from_bytes(data[:8], "little")
    if n > MAX_HEADER:
        return ("err", "exceeds the safety limit", None)
    if 8 + n > len(data):
        return ("err", "header extends beyond the file", None)
    try:
        text = data[8:8 + n].decode("utf-8")
        doc = json.loads(text, object_pairs_hook=_pairs, parse_int=_int, parse_float=_float,
                         parse_constant=_const)
        _check_tree(doc)
    except (_Reject, ValueError, RecursionError):
        return ("err", "must contain valid JSON", None)
    if not isinstance(doc, dict):
        return ("err", "must contain valid JSON", None)
    payload = len(data) - 8 - n
    out = {}
    for name in sorted(doc, key=lambda k: k.encode("utf-8")):
        if name == "__metadata__":
            continue
        t = doc[name]
        if not isinstance(t, dict):
            return ("err", "must be a JSON object, got", None)
        dt = t.get("dtype")
        if not isinstance(dt, str) or dt not in WIDTHS:
            return ("err", "unsupported dtype", name)
        sh = t.get("shape")
        if not isinstance(sh, list) or not all(_is_i64(d) and d >= 0 for d in sh):
            return ("err", "invalid shape", name)
        off = t.get("data_offsets")
        if (not isinstance(off, list) or len(off) != 2 or not all(_is_i64(o) for o in off)
                or off[0] < 0 or off[1] < off[0]):
            return ("err", "invalid data_offsets", name)
        if off[1] > payload:
            return ("err", "outside the file payload", name)
        count = 1
        for d in sh:
            count *= d
            if count >= 1 << 64:
                return ("err", "byte count mismatch", name)
        if (count * WIDTHS[dt]) % (1 << 64) != off[1] - off[0]:
            return ("err", "byte count mismatch", name)
        out[name] = (dt, list(sh), 8 + n + off[0], 8 + n + off[1])
    return ("ok", out)


# ------------------------------------------------------------------ seeds and mutations

def _file(header: bytes, payload: bytes) -> bytes:
    return len(header).to_bytes(8, "little") + header + payload


def _seeds():
    seeds = []
    h = {"__metadata__": {"format": "mlx", "note": "café \"q\" \\ /"},
         "model.layers.0.mlp.switch_mlp.gate_proj.weight": {"dtype": "U32", "shape": [4, 8, 2], "data_offsets": [0, 256]},
         "model.layers.0.mlp.switch_mlp.gate_proj.scales": {"dtype": "BF16", "shape": [4, 8, 1], "data_offsets": [256, 320]},
         "model.layers.0.mlp.switch_mlp.gate_proj.biases": {"dtype": "BF16", "shape": [4, 8, 1], "data_offsets": [320, 384]},
         "e": {"dtype": "F32", "shape": [], "data_offsets": [384, 388]},
         "z": {"dtype": "U8", "shape": [0, 7], "data_offsets": [388, 388]}}
    seeds.append(_file(json.dumps(h).encode(), bytes(388)))
    # escapes, astral characters, nested metadata, spacing and number spellings
    raw = ('{ "__metadata__" : {"a":[1,-2,3.5e-1,{"b":[[],{}]}],"c":null,"d":true,"f":false},\n'
           '\t"\\u00e9\\ud83d\\ude00\\n" : {"dtype":"I16","shape":[3 ,2],"data_offsets":[0,12]},\r'
           '"über\U0001f600" : {"shape":[1],"data_offsets":[12,13],"dtype":"BOOL"} }')
    seeds.append(_file(raw.encode("utf-8"), bytes(13)))
    # several tensors, an unsorted order (first error by name), padding spaces (as writers do)
    h = {f"t{i:02d}": {"dtype": "BF16", "shape": [i + 1, 2], "data_offsets": [4 * i * (i + 1) // 2, 4 * (i + 1) * (i + 2) // 2]}
         for i in reversed(range(6))}
    body = json.dumps(h).encode() + b" " * 13
    seeds.append(_file(body, bytes(84)))
    return seeds


TOKENS = [b"{", b"}", b"[", b"]", b'"', b"\\", b",", b":", b" ", b"\n", b"0", b"-", b".", b"e", b"E+",
          b"null", b"true", b"false", b"NaN", b"Infinity", b"\\u", b"\\ud800", b"\\udc00", b"\\u0000",
          b"\x00", b"\x1f", b"\x7f", b"\x80", b"\xc0\xaf", b"\xed\xa0\x80", b"\xf4\x90\x80\x80",
          b"\xe2\x82\xac", b"\xf0\x9f\x98\x80", b'"dtype"', b'"shape"', b'"data_offsets"',
          b'"__metadata__"', b'"U8"', b'"F64"', b"[0,0]", b"[]", b"{}"]
NUMBERS = [b"0", b"-0", b"-0.0", b"1", b"-1", b"9223372036854775807", b"9223372036854775808",
           b"-9223372036854775808", b"-9223372036854775809", b"18446744073709551615",
           b"18446744073709551616", b"4294967296", b"1e2", b"1.0", b"1e308", b"1.8e308", b"1e400",
           b"-1e400", b"1e-400", b"00", b"01", b"1" * 400, b"2147483648"]


def _mutate(rng: random.Random, data: bytes) -> bytes:
    n = int.from_bytes(data[:8], "little")
    head, tail = bytearray(data[8:8 + n]), data[8 + n:]
    framing = None
    for _ in range(rng.randint(1, 3)):
        op = rng.randrange(10)
        L = len(head)
        i = rng.randrange(L + 1)
        if op == 0 and L:
            head[min(i, L - 1)] = rng.randrange(256)
        elif op == 1:
            head[i:i] = rng.choice(TOKENS)
        elif op == 2 and L:
            del head[i:i + rng.randint(1, 8)]
        elif op == 3 and L:
            j = rng.randrange(L)
            head[i:i] = head[j:j + rng.randint(1, 24)]
        elif op == 4 and L > 2:
            a, b = sorted(rng.sample(range(L), 2))
            w = rng.randint(1, min(8, L - b))
            head[a:a + w], head[b:b + w] = head[b:b + w], head[a:a + w]
        elif op == 5:  # a number literal -> an edge value
            spans = [k for k in range(L) if chr(head[k]).isdigit() and (k == 0 or not chr(head[k - 1]).isdigit())]
            if spans:
                k = rng.choice(spans)
                e = k
                while e < L and chr(head[e]).isdigit():
                    e += 1
                head[k:e] = rng.choice(NUMBERS)
        elif op == 6:  # a shape whose element count overflows 64 bits
            k = head.find(b'"shape":')
            if k >= 0:
                e = head.find(b"]", k)
                if e > 0:
                    dims = rng.choice([b"[4294967296,4294967296]", b"[4294967296,4294967296,0]",
                                       b"[9223372036854775807,2]", b"[0,9223372036854775807,3]",
                                       b"[3037000500,3037000500]", b"[1,1,1,1,1,1,1,1,1,2]"])
                    head[k + 8:e + 1] = dims
        elif op == 7:  # header length prefix moved
            framing = max(0, n + rng.choice([-16, -3, -1, 1, 2, 7, 64]))
        elif op == 8:  # truncated file
            tail = tail[: rng.randrange(len(tail) + 1)]
        else:  # duplicate a key
            k = head.find(b'"', rng.randrange(L + 1))
            e = head.find(b'":', k + 1) if k >= 0 else -1
            if k >= 0 and e > k:
                head[k:k] = head[k:e + 2] + b"1,"
    length = len(head) if framing is None else framing
    return length.to_bytes(8, "little") + bytes(head) + tail


# ------------------------------------------------------------------ the comparison

def _library(path, name):
    try:
        e = P.safetensors_tensor(path, name)
    except AstroMoeError as err:
        assert err.status == INVALID_ARGUMENT, (name, str(err))
        return ("err", str(err))
    return ("ok", (e["dtype"], e["shape"], e["data_start_offset"], e["data_end_offset"]))


def _compare(path, data, case):
    want = model_parse(data)
    if want[0] == "err":
        _, cls, tensor = want
        got = _library(path, "model.layers.0.mlp.switch_mlp.gate_proj.weight")
        assert got[0] == "err", (case, want, got)
        assert cls in got[1], (case, want, got)
        if tensor is not None and "\x00" not in tensor:
            assert f'tensor "{tensor}"' in got[1], (case, want, got)
        return "err"
    entries = want[1]
    for name, (dt, shape, start, end) in entries.items():
        if "\x00" in name:
            continue
        got = _library(path, name)
        assert got == ("ok", (dt, shape[:8], start, end)), (case, name, want, got)
    got = _library(path, "not.a.tensor.in.this.header")
    assert got[0] == "err" and "is not in the safetensors header" in got[1], (case, got)
    return "ok"


def test_model_accepts_the_seeds():
    for s in _seeds():
        assert model_parse(s)[0] == "ok"


def test_fuzzed_headers_match_the_model(tmp_path):
    rng = random.Random(0x5AFE7E)
    seeds = _seeds()
    path = os.path.join(str(tmp_path), "case.safetensors")
    verdicts = {"ok": 0, "err": 0}
    cases = int(os.environ.get("ASTRO_FUZZ_CASES", "2500"))
    for case in range(cases):
        data = _mutate(rng, rng.choice(seeds))
        with open(path, "wb") as f:
            f.write(data)
        verdicts[_compare(path, data, case)] += 1
    # the mutations reach both sides of the checks
    assert verdicts["ok"] > cases // 50 and verdicts["err"] > cases // 2, verdicts


@pytest.mark.parametrize("depth,ok", [(126, True), (127, True), (128, False), (129, False), (5000, False)])
def test_nesting_limit(tmp_path, depth, ok):
    meta = b"[" * (depth - 1) + b"]" * (depth - 1)  # inside the top-level object: depth containers
    header = b'{"__metadata__":' + meta + b',"a":{"dtype":"U8","shape":[1],"data_offsets":[0,1]}}'
    path = os.path.join(str(tmp_path), "deep.safetensors")
    data = _file(header, b"\x00")
    open(path, "wb").write(data)
    assert (model_parse(data)[0] == "ok") == ok
    assert (_compare(path, data, depth) == "ok") == ok


def test_many_members_parse_quickly(tmp_path):
    # duplicate detection must not be quadratic in the number of entries
    n = 40000
    h = {f"t{i}": {"dtype": "U8", "shape": [1], "data_offsets": [i, i + 1]} for i in range(n)}
    path = os.path.join(str(tmp_path), "wide.safetensors")
    data = _file(json.dumps(h, separators=(",", ":")).encode(), bytes(n))
    open(path, "wb").write(data)
    t0 = time.perf_counter()
    assert _library(path, f"t{n - 1}") == ("ok", ("U8", [1], 8 + len(data) - 8 - n + n - 1, 8 + len(data) - 8 - n + n))
    assert time.perf_counter() - t0 < 10.0


def test_first_bad_entry_by_name_is_reported(tmp_path):
    h = (b'{"zz":{"dtype":"F64","shape":[1],"data_offsets":[0,8]},'
         b'"aa":{"dtype":"U8","shape":[-1],"data_offsets":[0,1]}}')
    path = os.path.join(str(tmp_path), "order.safetensors")
    data = _file(h, bytes(8))
    open(path, "wb").write(data)
    assert model_parse(data) == ("err", "invalid shape", "aa")
    got = _library(path, "zz")
    assert got[0] == "err" and 'tensor "aa" has an invalid shape' in got[1]


def test_number_edge_cases(tmp_path):
    path = os.path.join(str(tmp_path), "num.safetensors")
    cases = [(b"-0", "invalid shape"), (b"1.0", "invalid shape"), (b"9223372036854775808", "invalid shape"),
             (b"1e400", "must contain valid JSON"), (b"18446744073709551616", "invalid shape")]
    for lit, cls in cases:
        h = b'{"a":{"dtype":"U8","shape":[' + lit + b'],"data_offsets":[0,0]}}'
        data = _file(h, b"")
        open(path, "wb").write(data)
        assert model_parse(data)[:2] == ("err", cls), lit
        got = _library(path, "a")
        assert got[0] == "err" and cls in got[1], (lit, got)
    # an element count past 64 bits: a mismatch expecting 0 bytes
    h = b'{"a":{"dtype":"U8","shape":[4294967296,4294967296],"data_offsets":[0,0]}}'
    data = _file(h, b"")
    open(path, "wb").write(data)
    got = _library(path, "a")
    assert got[0] == "err" and "header declares 0 bytes but shape×dtype expects 0 bytes" in got[1], got
