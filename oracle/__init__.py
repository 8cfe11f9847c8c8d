"""CPU oracle for the KVMap-attention + KV-arena hot path.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import or run anything in this package,
and only as the checker (or the timed CPU baseline), never as the product
path. The product (cuda-kv-persistence_amd/, libkvpersist.so) never calls it.

Modules
  attention   fp32 explicit matmul+softmax restating the reference golden
              (reference: traces/gen_golden.py:30-74), plus a float64
              brute-force form for tiny shapes.
  policies    the five tile gating policies
              (reference: src/tile_gating_policy.cpp:1-83).
  manager     KVTileManager bookkeeping and the driver's per-frame plan
              (reference: src/kv_tile_manager.cu:12-219,
              src/run_policy_experiment.cu:136-283).
  trace_synth the reference's seeded synthetic trace generator, restated to
              regenerate the 8-frame seed-42 trace whose golden statistics
              the reference publishes (reference:
              traces/gen_synthetic_motion.py:41-89).
  backbone    the upstream K/V producer: LayerNorm, the q/k/v projections,
              the DiT block and the backbone forward in float64
              (reference: src/backbone.py:8-67).
  farneback   the upstream motion producer: OpenCV's Farneback dense flow
              restated from its published algorithm, the per-tile change
              rates and the trace post-processing
              (reference: traces/gen_motion_from_video.py:61-149).
  ref_build   recipe compiling the reference's own policy source into
              oracle/_ref/ (this container only; never shipped).

How each function is pinned (golden vectors, closed forms, reference build)
is stated in its module docstring.
"""
