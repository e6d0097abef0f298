"""CPU oracle for the fused RoPE + varlen attention path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this
package; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may use it, and only as the checker
(or, for ``cpu_baseline``, as the timed CPU port of the unfused path).

Contents (each function cites the reference file:line it restates):

* ``numerics``  -- bf16 / fp16 round-to-nearest-even emulation in numpy.
* ``rope``      -- ``compute_rope_2d`` (reference ``fused_attn.py:33-136``).
* ``windows``   -- ``get_window_index`` (reference ``utils.py:12-102``) and
  the per-frame ``cu_seqlens`` of full-attention layers.
* ``attention`` -- the unfused path: split-half rotation
  (``fused_attn.py:340-345,385-390``) followed by per-segment non-causal
  softmax attention (``fused_attn.py:347-423``), in fp32 (the official
  parity target), in a bf16-emulating variant that rounds at the same
  points as the fused kernel (``:344-345,389-390,413,423``), and a float64
  brute force for tiny inputs.

How each part is pinned (not by re-typing its own formula):

* rotation: closed-form invariants (norm preservation per pair, identity at
  cos=1/sin=0, composition of angles) and agreement with the HF
  ``rotate_half`` form; see ``tests/test_oracle.py``.
* attention: float64 brute force with explicit Python loops on tiny inputs,
  permutation equivariance inside a segment, shift invariance of logits,
  L=1 -> O=V, identical keys -> mean of V, segment independence.
* RoPE tables and window index: closed forms for single-axis grids and
  agreement with the third-party ``transformers`` implementation
  (``get_vision_position_ids``, ``Qwen2_5_VisionRotaryEmbedding``,
  ``get_vision_window_index``), plus committed golden fixtures under
  ``tests/golden/``.
"""
