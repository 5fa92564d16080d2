"""ORACLE -- test infrastructure only.

CPU restatements of the reference's population-forward path, used to check the product by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg. The product (noise_amd/) never imports, links or
runs anything here; there is no CPU fallback in the product.

  philox.c / noise.py   the noise draws (Philox4x32-10 under torch-ROCm's grid-stride layout), exact on
                        the integer side; pinned by published Random123 KATs and two independent
                        in-container implementations (oracle/crosscheck/).
  model.py              fp32 restatement of utils/model.py's forward and of eggroll.py's lowrank,
                        lowrank_embed and population_loss, and run.py's head_loss / hadamard draws.
"""
