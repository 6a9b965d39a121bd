"""OrcaSAQ-2-27B hot-path geometry, as the reference runtime fixes it
(model/footless/cuda_sm60/runtime.py:73-116), and the decode split policy
this build uses on MI355X."""

N_HEADS = 24            # full-attention q heads          runtime.py:78
N_KV = 4                # kv heads                        runtime.py:79
HEAD_DIM = 256          #                                 runtime.py:80
GQA_GROUP = N_HEADS // N_KV
ATTN_SCALE = HEAD_DIM ** -0.5                           # runtime.py:83
Q_PITCH = 2 * HEAD_DIM  # a head's row of the q|gate buffer: q(256) | gate(256) (kernels.cu:64-68)
GATE_OFF = HEAD_DIM

ROPE_DIM = 64           # partial rotary: the first 64 of 256 dims   runtime.py:81
ROPE_THETA = 1e7        #                                 runtime.py:82
NORM_EPS = 1e-6         # q / k RMSNorm (mean-space eps)   runtime.py:115

GDN_K_HEADS = 16        #                                 runtime.py:86
GDN_V_HEADS = 48        #                                 runtime.py:87
GDN_K = 128             #                                 runtime.py:88
GDN_V = 128             #                                 runtime.py:89
GDN_GROUP = GDN_V_HEADS // GDN_K_HEADS                  # runtime.py:90
CONV_WIDTH = 4          #                                 runtime.py:91
QKV_ROWS = 10240        # q(2048) | k(2048) | v(6144)      runtime.py:92-94
Q_SCALE = GDN_K ** -0.5                                 # runtime.py:101
L2_EPS = 1e-6           #                                 runtime.py:116
GDN_NORM_EPS = 1e-6     # GDN output RMSNormGated          runtime.py:113

# Decode / verify split policy on MI355X. A token's split count is
# clamp(max(seqlen / SPLIT_ROWS, min(seqlen / 64, 32)), 1, SPLIT_MAX): the
# reference's per-token rule (kernels.cu:535-544, with its ATT_SPLIT = 32 /
# ATT_GQA_ROWS = 32 of runtime.py:213-219 re-chosen) plus a floor of 32
# splits of 64 rows and up for short contexts (the library's batched decode
# applies it). At 4 sequences x 4 kv heads, 64 splits a long sequence give
# 1024 workgroups for 256 CUs, while a split keeps at least 256 rows (8
# tiles) so the partials stay a small fraction of the KV bytes (measured on
# MI355X: 256 beats 512 and 1024 at 8k / 32k contexts and ties at 100k); a
# 4k-row single sequence, 16 splits of 256 rows (64 workgroups), runs 1.3x
# faster as 32 splits of 128.
SPLIT_ROWS = 256
SPLIT_MAX = 64
# The batched decode's default: split_rows 0 asks the library for its grid
# rule instead -- floor(W / (B n_kv)) splits a token (W one workgroup a CU over
# fp16 caches, two over int8 ones; at most SPLIT_MAX, at least 64 rows a
# split), which beat the length rule at every batch size and context measured
# (B = 4, T = 3: ~8k 32.2 -> 29.5 us, ~32k 100.2 -> 87.7, ~100k 260.5 ->
# 245.7; B = 1 at ~8k 16.7 -> 14.4). Its split count depends on B, so a
# sequence's values in a batch can differ in the last bits from a
# single-sequence call's; SPLIT_ROWS keeps the length-only rule.
DEC_SPLIT_ROWS = 0
# The largest T the decode attention takes (MTP verify rows; runtime.py:299).
SPLIT_T_MAX = 4

GDN_CHUNK = 64

# The int8 KV cache (runtime.py:117-129): per position and kv head, 256 int8
# values and 8 fp16 block scales; a buffer of capacity max_pos holds all the
# values first, then all the scales.
KV8_BLOCK = 32
KV8_ROW = HEAD_DIM + 2 * (HEAD_DIM // KV8_BLOCK)   # bytes a position and kv head
# attention_dec_q8's split policy as the reference runtime sets it
# (runtime.py:219-220): at least DEC_TMIN 64-row tiles a split, at most
# DEC_SMAX splits.
DEC_TMIN = 1
DEC_SMAX = 28
LOG2E = 1.4426950408889634


def kv8_nbytes(max_pos: int, n_kv_heads: int = N_KV, head_dim: int = HEAD_DIM) -> int:
    """Bytes of one layer's int8 K (or V) buffer of capacity max_pos."""
    return max_pos * n_kv_heads * (head_dim + 2 * (head_dim // KV8_BLOCK))
