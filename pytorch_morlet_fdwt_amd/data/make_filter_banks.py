"""Regenerate ``filter_banks.json``: every discrete PyWavelets filter bank.

The package resolves wavelet names from this table, so PyWavelets is not needed at run
time.  Run with any interpreter that has PyWavelets installed::

    python make_filter_banks.py            # writes filter_banks.json next to this file

Each entry holds the four filters of ``pywt.Wavelet(name).filter_bank`` in PyWavelets'
order ``(dec_lo, dec_hi, rec_lo, rec_hi)``, written with ``repr`` so that every float
round-trips bit-exactly, plus the PyWavelets version that produced them.
"""

import json
import os

import pywt


def main():
    banks = {}
    for name in pywt.wavelist(kind="discrete"):
        w = pywt.Wavelet(name)
        banks[name] = [[float(v) for v in f] for f in w.filter_bank]
    out = {"pywt_version": pywt.__version__, "banks": banks}
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "filter_banks.json")
    with open(path, "w") as f:
        # repr() of a Python float is the shortest string that round-trips exactly
        f.write("{\n")
        f.write(f'  "pywt_version": {json.dumps(out["pywt_version"])},\n')
        f.write('  "banks": {\n')
        names = sorted(banks)
        for i, name in enumerate(names):
            rows = ", ".join("[" + ", ".join(repr(v) for v in flt) + "]" for flt in banks[name])
            f.write(f'    {json.dumps(name)}: [{rows}]' + (",\n" if i + 1 < len(names) else "\n"))
        f.write("  }\n}\n")
    print(f"wrote {len(banks)} filter banks to {path}")


if __name__ == "__main__":
    main()
