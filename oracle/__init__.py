"""ORACLE: CPU restatement of the reference sampling stage. Test infrastructure only
(tests/, __graft_entry__.smoke(), bench.py cpu_baseline); never the product path."""
