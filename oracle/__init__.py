"""CPU oracle of the shifted-window hot path (test infrastructure only).

Importable only from tests/, bench.py's cpu_baseline leg and
__graft_entry__.smoke(); the crumpet_amd package never imports it.
"""
