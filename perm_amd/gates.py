"""The byte-parity gate of the encode stage (coldpress/gates.py:34-58), on this
package's GGUF reader.

An encoded artifact may replace a stock quant only if a loader sees the same tensors
with the same container types and payload sizes: the final file must list exactly the
stock file's tensor names, each with the stock type and byte size, and its tensor bytes
may not exceed the stock total.
"""
from .ggufio import read_typemap


class GateError(AssertionError):
    """A hard gate failed."""


def _violations(final, stock):
    """Every way the final type map departs from the stock one, as readable lines."""
    out = [f"missing from the final artifact: {n}" for n in sorted(set(stock) - set(final))]
    out += [f"not in the stock artifact: {n}" for n in sorted(set(final) - set(stock))]
    for name in sorted(set(stock) & set(final)):
        for key in ("type", "n_bytes"):
            if final[name][key] != stock[name][key]:
                out.append(f"{name}: {key} {final[name][key]} (stock {stock[name][key]})")
    return out


def byte_parity(final_gguf, stock_gguf):
    """Check final_gguf against stock_gguf. Raises GateError listing what differs;
    returns {"tensors", "total_final", "total_stock", "passed": True} otherwise."""
    final, stock = read_typemap(final_gguf), read_typemap(stock_gguf)
    total_final = sum(v["n_bytes"] for v in final.values())
    total_stock = sum(v["n_bytes"] for v in stock.values())
    problems = _violations(final, stock)
    if total_final > total_stock:
        problems.append(f"tensor bytes {total_final} exceed the stock {total_stock}")
    if problems:
        shown = "; ".join(problems[:4]) + ("; ..." if len(problems) > 4 else "")
        raise GateError(f"byte parity: {len(problems)} violation(s): {shown}")
    return {"tensors": len(stock), "total_final": total_final, "total_stock": total_stock,
            "passed": True}
