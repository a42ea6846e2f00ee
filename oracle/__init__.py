"""CPU oracle for the Branchcraft hot path -- TEST INFRASTRUCTURE ONLY.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
as the checker; the product library never imports or links it."""
