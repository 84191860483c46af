"""PLY point clouds: a reader for every PLY encoding and a writer for scalar
elements.

The reference reads its dataset's ``points.ply`` with the third-party
``plyfile`` package (scripts/train_scanner_fixed.py:237-257); it is not a
dependency here.  ``read_ply`` parses the header itself (format
``ascii`` / ``binary_little_endian`` / ``binary_big_endian`` 1.0, elements,
scalar and list properties, comments) and returns, per element, one numpy
array per property.  Binary elements made only of scalar properties are read
as one structured view of the file (memory-mapped), so a point cloud of tens
of millions of vertices costs one pass over its bytes.
"""
from __future__ import annotations

import os
from typing import Dict, Iterable, List, Optional, Sequence, Tuple, Union

import numpy as np

__all__ = ["read_ply", "write_ply", "PlyError"]

_SCALAR = {
    "char": "i1", "int8": "i1", "uchar": "u1", "uint8": "u1",
    "short": "i2", "int16": "i2", "ushort": "u2", "uint16": "u2",
    "int": "i4", "int32": "i4", "uint": "u4", "uint32": "u4",
    "float": "f4", "float32": "f4", "double": "f8", "float64": "f8",
}
_NAME_OF = {"i1": "char", "u1": "uchar", "i2": "short", "u2": "ushort", "i4": "int",
            "u4": "uint", "f4": "float", "f8": "double"}
_FORMATS = {"ascii": None, "binary_little_endian": "<", "binary_big_endian": ">"}


class PlyError(ValueError):
    """Malformed or unsupported PLY file."""


# A property is (name, dtype) for a scalar or (name, (count dtype, item dtype)) for a list.
Prop = Tuple[str, Union[str, Tuple[str, str]]]


def _parse_header(buf: memoryview) -> Tuple[str, List[Tuple[str, int, List[Prop]]], int]:
    head = bytes(buf[: min(len(buf), 1 << 20)])
    end = head.find(b"end_header")
    if not head.startswith(b"ply") or end < 0:
        raise PlyError("not a PLY file (no 'ply' magic or no end_header)")
    eol = head.find(b"\n", end)
    body = (eol + 1) if eol >= 0 else len(head)  # the body starts after the end_header line
    lines = head[:end].decode("ascii", errors="replace").splitlines()
    fmt = None
    elements: List[Tuple[str, int, List[Prop]]] = []
    for raw in lines[1:]:
        tok = raw.split()
        if not tok or tok[0] in ("comment", "obj_info"):
            continue
        if tok[0] == "format":
            if len(tok) < 3 or tok[1] not in _FORMATS or tok[2] != "1.0":
                raise PlyError(f"unsupported PLY format line: {raw!r}")
            fmt = tok[1]
        elif tok[0] == "element":
            if len(tok) != 3:
                raise PlyError(f"bad element line: {raw!r}")
            elements.append((tok[1], int(tok[2]), []))
        elif tok[0] == "property":
            if not elements:
                raise PlyError("property before any element")
            if len(tok) == 5 and tok[1] == "list":
                if tok[2] not in _SCALAR or tok[3] not in _SCALAR:
                    raise PlyError(f"unknown list property types: {raw!r}")
                elements[-1][2].append((tok[4], (_SCALAR[tok[2]], _SCALAR[tok[3]])))
            elif len(tok) == 3:
                if tok[1] not in _SCALAR:
                    raise PlyError(f"unknown property type: {raw!r}")
                elements[-1][2].append((tok[2], _SCALAR[tok[1]]))
            else:
                raise PlyError(f"bad property line: {raw!r}")
        else:
            raise PlyError(f"unknown header line: {raw!r}")
    if fmt is None:
        raise PlyError("PLY header has no format line")
    return fmt, elements, body


def _read_binary(buf, off: int, order: str, count: int, props: List[Prop]):
    out: Dict[str, object] = {}
    if all(isinstance(t, str) for _, t in props):
        dt = np.dtype([(n, order + t) for n, t in props])
        need = dt.itemsize * count
        if off + need > len(buf):
            raise PlyError("PLY body shorter than its header declares")
        rec = np.frombuffer(buf, dtype=dt, count=count, offset=off)
        for n, _ in props:
            out[n] = rec[n].astype(rec[n].dtype.newbyteorder("="), copy=True)
        return out, off + need
    # elements with list properties: one row at a time
    cols: Dict[str, list] = {n: [] for n, _ in props}
    for _ in range(count):
        for n, t in props:
            if isinstance(t, str):
                d = np.dtype(order + t)
                if off + d.itemsize > len(buf):
                    raise PlyError("PLY body shorter than its header declares")
                cols[n].append(np.frombuffer(buf, dtype=d, count=1, offset=off)[0])
                off += d.itemsize
            else:
                cd, idt = np.dtype(order + t[0]), np.dtype(order + t[1])
                if off + cd.itemsize > len(buf):
                    raise PlyError("PLY body shorter than its header declares")
                k = int(np.frombuffer(buf, dtype=cd, count=1, offset=off)[0])
                off += cd.itemsize
                if k < 0 or off + k * idt.itemsize > len(buf):
                    raise PlyError("bad list length in PLY body")
                cols[n].append(np.frombuffer(buf, dtype=idt, count=k, offset=off)
                               .astype(idt.newbyteorder("=")))
                off += k * idt.itemsize
    for n, t in props:
        out[n] = np.array(cols[n], dtype=t) if isinstance(t, str) else cols[n]
    return out, off


def _read_ascii(tokens: List[bytes], pos: int, count: int, props: List[Prop]):
    out: Dict[str, object] = {}
    if all(isinstance(t, str) for _, t in props):
        k = len(props)
        if pos + count * k > len(tokens):
            raise PlyError("PLY body shorter than its header declares")
        block = np.array(tokens[pos: pos + count * k], dtype=object).reshape(count, k)
        for j, (n, t) in enumerate(props):
            kind = np.dtype(t).kind
            col = block[:, j].astype(np.float64 if kind == "f" else np.int64)
            out[n] = col.astype(t)
        return out, pos + count * k
    cols: Dict[str, list] = {n: [] for n, _ in props}
    for _ in range(count):
        for n, t in props:
            if isinstance(t, str):
                cols[n].append(float(tokens[pos]) if np.dtype(t).kind == "f" else int(tokens[pos]))
                pos += 1
            else:
                k = int(tokens[pos])
                pos += 1
                conv = float if np.dtype(t[1]).kind == "f" else int
                cols[n].append(np.array([conv(x) for x in tokens[pos: pos + k]], dtype=t[1]))
                pos += k
    for n, t in props:
        out[n] = np.array(cols[n], dtype=t) if isinstance(t, str) else cols[n]
    return out, pos


def read_ply(path: Union[str, os.PathLike], elements: Optional[Iterable[str]] = None
             ) -> Dict[str, Dict[str, object]]:
    """Elements of a PLY file: ``{element: {property: array}}``.  Scalar
    properties are numpy arrays in native byte order; list properties are
    lists of arrays.  ``elements`` limits the result (parsing stops after the
    last requested element)."""
    want = None if elements is None else set(elements)
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    buf = memoryview(mm)
    fmt, header, off = _parse_header(buf)
    result: Dict[str, Dict[str, object]] = {}
    if fmt == "ascii":
        tokens = bytes(buf[off:]).split()
        pos = 0
        for name, count, props in header:
            if want is not None and not (want - set(result)):
                break
            data, pos = _read_ascii(tokens, pos, count, props)
            if want is None or name in want:
                result[name] = data
    else:
        order = _FORMATS[fmt]
        for name, count, props in header:
            if want is not None and not (want - set(result)):
                break
            data, off = _read_binary(mm, off, order, count, props)
            if want is None or name in want:
                result[name] = data
    if want is not None and want - set(result):
        raise PlyError(f"PLY file has no element(s) {sorted(want - set(result))}")
    return result


def write_ply(path: Union[str, os.PathLike], elements: Dict[str, Dict[str, np.ndarray]],
              fmt: str = "binary_little_endian", comments: Sequence[str] = ()) -> None:
    """Write scalar-property elements (``{element: {property: 1-D array}}``,
    insertion order kept) in ``ascii`` or either binary encoding."""
    if fmt not in _FORMATS:
        raise PlyError(f"unknown PLY format {fmt!r}")
    lines = ["ply", f"format {fmt} 1.0"] + [f"comment {c}" for c in comments]
    blocks = []
    for name, props in elements.items():
        cols = [np.asarray(v) for v in props.values()]
        n = len(cols[0]) if cols else 0
        if any(c.ndim != 1 or len(c) != n for c in cols):
            raise PlyError(f"element {name!r}: properties must be 1-D arrays of one length")
        lines.append(f"element {name} {n}")
        fields = []
        for pname, c in zip(props.keys(), cols):
            code = c.dtype.str[1:]
            if code not in _NAME_OF:
                raise PlyError(f"property {pname!r}: dtype {c.dtype} has no PLY type")
            lines.append(f"property {_NAME_OF[code]} {pname}")
            fields.append((pname, code))
        blocks.append((fields, cols, n))
    lines.append("end_header")
    with open(path, "wb") as f:
        f.write(("\n".join(lines) + "\n").encode("ascii"))
        for fields, cols, n in blocks:
            if fmt == "ascii":
                for i in range(n):
                    f.write((" ".join(repr(float(c[i])) if c.dtype.kind == "f" else str(int(c[i]))
                                      for c in cols) + "\n").encode("ascii"))
            else:
                order = _FORMATS[fmt]
                rec = np.empty(n, dtype=np.dtype([(p, order + t) for p, t in fields]))
                for (p, _), c in zip(fields, cols):
                    rec[p] = c
                f.write(rec.tobytes())
