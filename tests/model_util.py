"""Order / User records as Python dicts <-> ModelColumns (test helper)."""
import numpy as np

import petjson as pj

MODELS = {"order": pj.MODEL_ORDER, "user": pj.MODEL_USER}


def to_model_columns(model: int, records) -> pj.ModelColumns:
    """Host columns from dicts (a missing or None property is null)."""
    props = pj.MODEL_PROPS[model]
    n = len(records)
    present = np.zeros(n, np.uint8)
    col, byt = [], []
    for k, (name, kind) in enumerate(props):
        vals = [r.get(name) for r in records]
        for i, v in enumerate(vals):
            if v is not None:
                present[i] |= 1 << k
        if kind == "str":
            bs = [v.encode("utf-8") if isinstance(v, str) else (v or b"") for v in vals]
            off = np.zeros(n + 1, np.uint64)
            off[1:] = np.cumsum([len(b) for b in bs], dtype=np.uint64) if n else []
            col.append(off)
            byt.append(np.frombuffer(b"".join(bs), np.uint8).copy())
        elif kind == "enum":
            col.append(np.array([pj.ORDER_STATUS.index(v) if v is not None else 0 for v in vals], np.uint8))
            byt.append(None)
        elif kind == "bool":
            col.append(np.array([1 if v else 0 for v in vals], np.uint8))
            byt.append(None)
        else:
            col.append(np.array([v or 0 for v in vals], pj.KIND_DTYPE[kind]))
            byt.append(None)
    return pj.ModelColumns(model, n, present, col, byt)


def from_model_columns(c: pj.ModelColumns):
    """Dicts of the non-null properties of each record (strings as str when
    they are UTF-8, else bytes)."""
    c = c.to_host() if not isinstance(c.col[0], np.ndarray) else c
    out = []
    for i in range(c.n):
        r = {}
        for k, (name, kind) in enumerate(c.props):
            if c.present is not None and not (int(c.present[i]) >> k) & 1:
                continue
            v = c.col[k]
            if kind == "str":
                b = c.bytes[k][int(v[i]): int(v[i + 1])].tobytes()
                try:
                    r[name] = b.decode("utf-8")
                except UnicodeDecodeError:
                    r[name] = b
            elif kind == "enum":
                r[name] = pj.ORDER_STATUS[int(v[i])]
            elif kind == "bool":
                r[name] = bool(v[i])
            else:
                r[name] = int(v[i])
        out.append(r)
    return out
