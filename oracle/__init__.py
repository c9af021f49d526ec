"""CPU oracle (test infrastructure only — never imported by the product).

See ``oracle/svdq_oracle.py`` for what it restates and how it is pinned.
"""
