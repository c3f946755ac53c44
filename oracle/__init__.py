"""CPU oracle for the MoE-layer hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker / the timed CPU baseline. The product
path (glmserve_amd) never imports it.

Two libraries are wrapped:
  * libmoe_oracle.so -- this build's C restatement (oracle/moe_oracle.c);
  * libglmref.so     -- glmserve's own CPU MoE path (GLM52Model::moe_mlp,
                        src/model_glm52.cpp:1096-1154) compiled from the
                        reference sources by oracle/Makefile (optional: only
                        present where the reference tree was available at
                        build time).
"""
from .pyoracle import (Oracle, RefLib, build, load_oracle, load_ref, ORACLE_SO, REF_SO)  # noqa: F401
