"""CPU oracle of the product-key-memory lookup: test infrastructure only (tests/, __graft_entry__.smoke(),
bench.py cpu_baseline).  The product (sparse-memory-lm_amd/smlm_hip) never imports it."""
