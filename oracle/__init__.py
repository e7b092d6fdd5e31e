"""CPU oracle for the Qorus-IA quantized matrix path.

Test infrastructure only: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker.  The shipped library
(project-ia_amd/) never imports, links or calls anything in this package.
"""
