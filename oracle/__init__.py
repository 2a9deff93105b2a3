"""CPU oracle (test infrastructure only; never imported by the product path).

See ``oracle/quant_ref.py`` for the restated reference functions.
"""
