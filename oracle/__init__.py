"""CPU oracle of agent-factory-3's MXFP4 MoE expert path — TEST INFRASTRUCTURE ONLY.

Plain numpy / torch-CPU restatements of the reference's algorithms, each
function citing the reference file:line it follows (paths relative to
``src/agent_factory_3/models/gpt_oss/`` unless stated).  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only as the checker / the reported CPU baseline: the product
path (``agent_factory_3_amd``) never calls it.

How each part is pinned (no reference golden vectors exist for this path):

* ``mxfp4``   — integer bit formula (kernels.py:120-158) checked against an
  independent LUT + ldexp restatement (quantization.py:102-122) over all
  16 nibbles x 256 scale bytes where both are defined, against exact
  rational arithmetic (value = e2m1 * 2^(S-127)) for every pair, and against
  the committed exhaustive table ``tests/golden/mxfp4_table.npy``.
* ``swiglu``  — closed form (kernels.py:431-441, 533-545) checked against
  float64 torch autograd of the clamp/sigmoid expression with the strict
  masks, plus special points (g = limit, u = +-limit, saturated sigmoid).
* ``routing`` — routing_replay / top-k restated with torch CPU ops
  (quantization.py:551-636) and checked by invariants (inverse permutation,
  histogram sum, stability, per-token weights summing to 1) and brute force.
* ``moe``     — per-expert fp32 loops (matmul_ogs semantics as called at
  quantization.py:358-362, 409-418), checked against float64 brute force
  on tiny shapes and against the dense mathematical layer
  (routing -> gather -> GEMM -> SwiGLU -> GEMM -> gamma-weighted sum).
* ``lora``    — closed forms of the expert-LoRA gradients checked against
  float64 torch autograd of the restated forward.
"""
