"""Module-global knobs of the delta-attention path, with the reference's names and defaults.

Mirrors the hot-path knobs of globVR.py (lines 42, 65-70, 79, 83-92) and the ones the
reference reads with getattr defaults (modeling_llama.py:583, 716, 1176).  Set them
with ``setattr(globVR, name, value)`` exactly as the reference's harnesses do
(eval_speedup.py:47-68).

Only the exact string "cosine" selects the cosine metric (modeling_llama.py:639-640);
every other value of ``row_similarity_metric`` ("cos", "euclidian", ...) is Euclidean.
"""

# prefill delta path switch (modeling_llama.py:600)
delta_pf_key_on = 1
delta_type = "regular"          # "row" enables the delta prefill path

# anchor selection (modeling_llama.py:602-653)
row_delta_threshold = 10
row_similarity_metric = "cos"
divide_to = 1
chunk_size = 0                  # 0 = use divide_to; >0 = fixed tokens per chunk
packing_mode = "delta"          # "delta" | "random" | "periodic"
row_delta_arith = "native"      # Euclidean distance in the keys' "native" 16-bit arithmetic
                                # (tritonModules.py:55-58) or in "fp32"
target_keep_rate = 0.5          # used by the random and periodic packing modes

# hybrid kernel variants (modeling_llama.py:716-749)
dense_window_size = 128
sanity = False                  # Phase 1 decides the window start but adds nothing
no_count = False                # every count (padding included) is 1
pure_phase1 = False             # packed history only, no dense window

# dense control and decoding (modeling_llama.py:778, 536, 805)
flash = False
delta_decode = False
kv_log_interval = 10
skip_causal_mask = False

# timing and bookkeeping (modeling_llama.py:533, 694-698; glob_set.py:32-66)
time_internal = True
spars = 0.0
latency_stats = {}
latency_events = []
kv_compression_samples = []
