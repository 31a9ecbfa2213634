"""The byte-parity gate of coldpress/gates.py:34-58 on this package's GGUF reader."""
from .ggufio import read_typemap


class GateError(AssertionError):
    pass


def byte_parity(final_gguf, stock_gguf):
    """The final artifact has the stock quant's per-tensor type map and sizes and no more
    total tensor bytes. Raises GateError otherwise; returns a report dict."""
    fm = read_typemap(final_gguf)
    sm = read_typemap(stock_gguf)
    if set(fm) != set(sm):
        only_final = sorted(set(fm) - set(sm))
        only_stock = sorted(set(sm) - set(fm))
        raise GateError(f"byte-parity FAIL: tensor-set differs "
                        f"(+final {only_final[:4]}, +stock {only_stock[:4]})")
    mismatches = []
    for name in sm:
        if fm[name]["type"] != sm[name]["type"]:
            mismatches.append((name, "type", fm[name]["type"], sm[name]["type"]))
        if fm[name]["n_bytes"] != sm[name]["n_bytes"]:
            mismatches.append((name, "n_bytes", fm[name]["n_bytes"], sm[name]["n_bytes"]))
    total_final = sum(v["n_bytes"] for v in fm.values())
    total_stock = sum(v["n_bytes"] for v in sm.values())
    if mismatches:
        raise GateError(f"byte-parity FAIL: {len(mismatches)} per-tensor mismatches, "
                        f"e.g. {mismatches[:3]}")
    if total_final > total_stock:
        raise GateError(f"byte-parity FAIL: total {total_final} > stock {total_stock}")
    return {"tensors": len(sm), "total_final": total_final, "total_stock": total_stock,
            "passed": True}
