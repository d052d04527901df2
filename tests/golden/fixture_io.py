"""Fixture format: one .npz per case.

Tables are stored sparsely (only the rows a case touches, the others are zero) so that a fixture
can keep the vocabulary size, and therefore the clamp bound, of the case it records.
Keys: values, offsets, batch, [val_base], table_dtype, out_dtype, pooling, expected,
      num_tables, shared, and per table i: t{i}_shape (V, D), t{i}_rows, t{i}_data.
"""
import numpy as np


def save(path, values, offsets, batch, tables, table_dtype, out_dtype, pooling, expected, val_base=None,
         shared=False):
    d = dict(values=np.asarray(values, np.int64), offsets=np.asarray(offsets, np.int64), batch=np.int64(batch),
             table_dtype=np.str_(table_dtype), out_dtype=np.str_(out_dtype), pooling=np.str_(pooling),
             expected=expected, shared=np.int64(shared))
    if val_base is not None:
        d["val_base"] = np.asarray(val_base, np.int64)
    store = tables[:1] if shared else tables
    d["num_tables"] = np.int64(len(store))
    for i, t in enumerate(store):
        nz = np.flatnonzero(np.any(t != 0, axis=1))
        d[f"t{i}_shape"] = np.array(t.shape, np.int64)
        d[f"t{i}_rows"] = nz.astype(np.int64)
        d[f"t{i}_data"] = t[nz]
    np.savez_compressed(path, **d)


def load(path, num_fields=None):
    z = np.load(path, allow_pickle=False)
    out = {k: z[k] for k in ("values", "offsets", "expected")}
    out["batch"] = int(z["batch"])
    for k in ("table_dtype", "out_dtype", "pooling"):
        out[k] = str(z[k])
    out["val_base"] = z["val_base"] if "val_base" in z.files else None
    tables = []
    for i in range(int(z["num_tables"])):
        V, D = (int(x) for x in z[f"t{i}_shape"])
        data = z[f"t{i}_data"]
        t = np.zeros((V, D), dtype=data.dtype)
        t[z[f"t{i}_rows"]] = data
        tables.append(t)
    if int(z["shared"]):
        F = len(out["val_base"]) if out["val_base"] is not None else num_fields
        tables = tables * F
    out["tables"] = tables
    out["shared"] = bool(int(z["shared"]))
    return out
