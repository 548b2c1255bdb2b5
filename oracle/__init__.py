"""CPU oracle: a PyTorch-fp32 (and fp64 for brute force) restatement of the
reference's one-step recurrent inference path, used ONLY as the checker.

TEST INFRASTRUCTURE. Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import anything from here, and only to
check or time against it. The product (`hackathon_amd/`) never imports it.

Modules
- `oracle.kernels`  the three fused state steps (model/kernels.py:124-171).
- `oracle.model`    the 4-tower ensemble forward/init_state
                    (model/inference_model.py, model/{modules,mamba2,retnet,
                    hawk,xlstm}.py) and CastLinear semantics
                    (example_model.py:68-148).
- `oracle.client`   process_batch round splitting and row assignment
                    (example_model.py:724-905).
- `oracle.init`     numpy restatement of the deterministic init spec, used to
                    pin the library's fast generator.

How each part is pinned is recorded in tests/ (see tests/test_oracle_*.py).
"""
