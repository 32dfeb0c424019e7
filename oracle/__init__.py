"""CPU oracle for the YOLO frame path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference's arithmetic on the CPU in numpy fp32 so the HIP
engine can be checked against it.  Only `tests/`, `__graft_entry__.smoke()` and
`bench.py`'s `cpu_baseline` leg may import it, and only as the checker (or as the timed
CPU baseline).  The engine library never links, loads or calls anything here, and the
product path has no CPU fallback.

Modules:
  graphfile  model.graph / weights.f16 / bias.f32 reader   (engine/engine.cu:88-248)
  interp     fp32 per-op graph interpreter                  (export/export.py:446-526)
  post       letterbox, DFL decode, NMS, masks, probiou     (engine/engine.cu:844-1252)

Pinning (what checks each function, beyond re-typing its formula) is listed in the
header of each module; every function is pinned, none is "parity unpinned" except where
a module header says so.
"""
