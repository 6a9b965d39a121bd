"""The C ABI on the CPU: libfl355.so loads without a GPU, exports every
entry point include/fl355.h declares, and its argument checks refuse bad
geometry before anything is launched (no device call is made by these)."""
import ctypes
import re
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent


def declared_entry_points():
    text = (REPO / "include" / "fl355.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(fl_\w+)\(", text, re.M)))


def test_header_declares_the_path():
    names = declared_entry_points()
    for want in ("fl_kv_store", "fl_attention_split_gqa", "fl_attention_merge", "fl_attn_gate",
                 "fl_attn_decode", "fl_attention_prefill", "fl_conv1d_causal",
                 "fl_conv1d_causal_rows", "fl_l2norm_scaled", "fl_gdn_scalars", "fl_gdn_scan",
                 "fl_gdn_decode", "fl_gdn_prefill_chunked"):
        assert want in names


def test_library_exports_every_declared_symbol(fl):
    lib = fl._lib.lib()
    missing = [n for n in declared_entry_points() if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding covers every one of them
    assert set(declared_entry_points()) <= set(fl._lib.SIGNATURES)


def test_op_layer_fails_loudly_without_the_library(tmp_path):
    """With libfl355.so absent the op layer raises instead of computing
    anything another way (there is no CPU path), in a fresh process so the
    library this session loaded stays in place."""
    import subprocess
    import sys
    code = (
        "import sys; from pathlib import Path\n"
        f"sys.path.insert(0, {str(REPO)!r})\n"
        "import __graft_entry__ as ge\n"
        "fl = ge.load_package()\n"
        "fl._lib._lib = None\n"
        f"fl._lib.LIB_PATH = Path({str(tmp_path / 'absent.so')!r})\n"
        "try:\n"
        "    fl.ops.prefill_split_count(1024, 98000)\n"
        "except ImportError as e:\n"
        "    print('raised:', e)\n"
        "    sys.exit(0)\n"
        "sys.exit(3)\n")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "absent.so is missing" in r.stdout


def test_status_strings(fl):
    lib = fl._lib.lib()
    assert lib.fl_abi_version() == 1
    assert lib.fl_strerror(0) == b"ok"
    assert lib.fl_strerror(1) == b"invalid argument"


def _call(fl, name, *args):
    return getattr(fl._lib.lib(), name)(*args)


def test_argument_checks_refuse_before_launch(fl):
    lib = fl._lib.lib()
    fake = ctypes.c_void_p(0x1000)   # never dereferenced: every call below fails its checks
    # kv_store past the cache end
    assert _call(fl, "fl_kv_store", fake, fake, fake, fake, 0, 10, 5, 4, 256, 12, None) == 1
    assert b"max_pos" in lib.fl_last_error()
    # decode: 6 tokens x 6 heads > 32 columns
    assert _call(fl, "fl_attention_split_gqa", fake, fake, fake, fake, fake, fake, 0, 24, 4, 256,
                 512, 0, 100, 0.0625, 512, 6, 8, None) == 1
    # head_dim other than 256
    assert _call(fl, "fl_attention_prefill", fake, 128, None, None, fake, fake, 0, 24, 4, 128, 0,
                 64, 1.0, 8, fake, 128, None) == 1
    # conv with aliased state buffers
    assert _call(fl, "fl_conv1d_causal", fake, fake, fake, fake, fake, 64, 1, 1, 64, 4, None) == 1
    assert b"distinct" in lib.fl_last_error()
    # scan with K != 128
    assert _call(fl, "fl_gdn_scan", fake, fake, fake, fake, fake, fake, fake, 4, 16, 48, 64, 128,
                 10240, 10240, 6144, 0.1, 3, None, 0, None) == 1
    # chunked scan with a chunk other than 64
    assert _call(fl, "fl_gdn_prefill_chunked", fake, fake, fake, fake, fake, fake, fake, 100, 16,
                 48, 128, 128, 10240, 10240, 6144, 0.1, 3, 32, fake, 1 << 30, None) == 1
    # the chunked scan from logits without A_log, or with a logit row shorter
    # than the v heads
    assert _call(fl, "fl_gdn_prefill_chunked_logits", fake, fake, fake, fake, fake, 48, None,
                 fake, fake, fake, 100, 16, 48, 128, 128, 10240, 10240, 6144, 0.1, 3, 64, fake,
                 1 << 30, None) == 1
    assert _call(fl, "fl_gdn_prefill_chunked_logits", fake, fake, fake, fake, fake, 40, fake,
                 fake, fake, fake, 100, 16, 48, 128, 128, 10240, 10240, 6144, 0.1, 3, 64, fake,
                 1 << 30, None) == 1
    assert b"ab_stride" in lib.fl_last_error()
    # the gated prefill needs q | gate rows (q_pitch >= 2 head_dim)
    assert _call(fl, "fl_attention_prefill_gated", fake, 256, None, None, fake, fake, 0, 0, 24, 4,
                 256, 0, 64, 1.0, 8, 1, fake, 256, None, 0, None) == 1
    assert b"gate" in lib.fl_last_error()
    # batched prep: no rows, more rows than FL_MAX_SEQS, a row past its capacity
    arr = fl._lib.ptr_array([0x2000] * 17)
    pos, caps = fl._lib.int_array([5] * 17), fl._lib.int_array([8] * 17)
    for B in (0, 17):
        assert _call(fl, "fl_attn_prep_rows", fake, 512, fake, fake, fake, fake, arr, arr, pos,
                     caps, B, 0, 24, 4, 256, 64, 1e7, 1e-6, None) == 1
    over = fl._lib.int_array([8] + [5] * 16)
    assert _call(fl, "fl_attn_prep_rows", fake, 512, fake, fake, fake, fake, arr, arr, over, caps,
                 2, 1, 24, 4, 256, 64, 1e7, 1e-6, None) == 1
    assert b"max_pos" in lib.fl_last_error()
    # decode + output norm: V other than 128, more rows than FL_MAX_SEQS, a
    # sequence's two conv buffers aliased, an odd z pitch
    pp = fl._lib.ptr_array([0x2000] * 17)
    pq = fl._lib.ptr_array([0x3000] * 17)
    p0 = fl._lib.int_array([5] * 17)

    def normed(B, V, cin, z_pitch, T=1, conv=1):
        return _call(fl, "fl_gdn_decode_normed", fake, 10240, conv, fake, cin, pq, p0, fake, fake,
                     48, fake, fake, pp, None, 0, fake, z_pitch, fake, fake, 6144, B, T, 16, 48,
                     128, V, 0.088, 1e-6, 1e-6, None)
    assert normed(4, 64, pp, 6144) == 1
    assert normed(17, 128, pp, 6144) == 1
    assert normed(2, 128, pq, 6144) == 1 and b"distinct" in lib.fl_last_error()
    assert normed(2, 128, pp, 6145) == 1 and b"pitch" in lib.fl_last_error()
    assert normed(1, 128, pp, 6144, T=4, conv=0) == 1 and b"T <= 3" in lib.fl_last_error()
    assert normed(1, 128, pp, 6144, T=3, conv=1) == 1 and b"conv_fused" in lib.fl_last_error()


def test_work_size_queries(fl):
    lib = fl._lib.lib()
    assert lib.fl_attn_decode_work_bytes(4, 3, 24, 256, 64) == 4 * 3 * 24 * 64 * (256 + 2) * 4
    # per (chunk, v head): T and M o QK^T as hi / lo fp16 MFMA operands of
    # their 6 nonzero 16 x 32 blocks (4 x 6 x 16 x 32 x 2 bytes: both are lower
    # triangular, the blocks above the diagonal are left out), beta / e^g /
    # e^{g_C - g} (3 x 64 f32) and a 64-float block of scalars
    n_chunks = (8192 + 63) // 64
    assert lib.fl_gdn_chunked_work_bytes(8192, 48, 128, 128, 64) == \
        n_chunks * 48 * (4 * 6 * 16 * 32 * 2 + 4 * 64 * 4)
    assert lib.fl_gdn_chunked_work_bytes(8192, 48, 128, 128, 32) == 0


def test_scratch_too_small_is_reported(fl):
    fake = ctypes.c_void_p(0x1000)
    arr = fl._lib.ptr_array([0x2000])
    ints = fl._lib.int_array([100])
    caps = fl._lib.int_array([200])
    rc = _call(fl, "fl_attn_decode", fake, 512, arr, arr, ints, caps, 1, 1, 24, 4, 256, 0.0625,
               512, 64, None, 512, 256, fake, 256, fake, 16, None)
    assert rc == 3 and b"work" in fl._lib.lib().fl_last_error()


def test_op_layer_refuses_cpu_tensors(fl):
    torch = pytest.importorskip("torch")
    k = torch.zeros((1, 4, 256), dtype=torch.float16)
    with pytest.raises(ValueError):
        fl.ops.kv_store(k, k, torch.zeros((8, 4, 256), dtype=torch.float16),
                        torch.zeros((8, 4, 256), dtype=torch.float16), pos0=0)


def test_noalloc_decode_refuses_beyond_its_static_scratch(fl):
    """fl_attn_decode_noalloc checks the partials' size against its static
    array before anything touches the device."""
    lib = fl._lib.lib()
    assert lib.fl_attn_decode_noalloc_max_bytes() == 32 << 20
    need = lib.fl_attn_decode_work_bytes(16, 5, 24, 256, 64)
    assert need > lib.fl_attn_decode_noalloc_max_bytes()
    fake = ctypes.c_void_p(0x1000)
    arr = fl._lib.ptr_array([0x1000] * 16)
    ints = fl._lib.int_array([100] * 16)
    rc = _call(fl, "fl_attn_decode_noalloc", fake, 512, arr, arr, ints, ints, 16, 5, 24, 4, 256,
               0.0625, 256, 64, None, 512, 256, fake, 256, None)
    assert rc == 3                                  # FL_ESCRATCH
    assert b"static scratch" in lib.fl_last_error()


def test_prefill_split_policy(fl):
    """The KV split the prefill takes: none where the grid fills the CUs (an 8k
    or 2k fresh prompt, a 4k chunk deep in a prompt: the 64-rows-a-wave kernel
    or 384+ workgroups of 128 rows), 8 for the reference's 1024-token chunk at
    pos0 98k (192 workgroups of 128 rows on 256 CUs; the 64-rows-a-wave
    kernel's 96 a split x 8 = 3 rounds), 8 for a 512-token chunk (the 128-row
    kernel's split); the work it needs."""
    lib = fl._lib.lib()
    assert lib.fl_attention_prefill_split_count(8192, 0, 24, 4) == 1
    assert lib.fl_attention_prefill_split_count(2048, 0, 24, 4) == 1
    assert lib.fl_attention_prefill_split_count(4096, 98000, 24, 4) == 1
    assert lib.fl_attention_prefill_split_count(1024, 98000, 24, 4) == 8
    assert lib.fl_attention_prefill_split_count(512, 98000, 24, 4) == 8
    # over an int8 cache the 128-row int8 kernel always runs: its own cost model
    assert lib.fl_attention_prefill_split_count_q8(1024, 98000, 24, 4) == 4
    assert lib.fl_attention_prefill_split_count_q8(512, 98000, 24, 4) == 8
    assert lib.fl_attention_prefill_split_count_q8(8192, 0, 24, 4) == 1
    assert lib.fl_attention_prefill_work_bytes(1024, 24, 256, 4) == 1024 * 24 * 4 * (256 * 4 + 8)
    assert lib.fl_attention_prefill_work_bytes(1024, 24, 256, 1) == 0



def _plan_weights(T, pos0, G):
    RT = T * G
    N = (RT + 255) // 256
    return [(pos0 + min(t * 256 + 255, RT - 1) // G + 1 + 31) // 32 + 5 for t in range(N)]


@pytest.mark.parametrize("T,pos0", [(6144, 0), (8192, 0), (12288, 0), (32768, 0), (8192, 20000)])
def test_prefill_persistent_plan(fl, T, pos0):
    """The persistent plan of the long-prefill kernel on 256 CUs: every 256-row
    tile of a kv head in exactly one of the 64 bins, each bin heaviest first,
    and the heaviest bin within 4 % of the bound max(mean load, heaviest
    tile) -- greedy longest-first alone is 10 % over it at T = 8192."""
    lib = fl._lib.lib()
    buf = (ctypes.c_ushort * 1024)()
    n = lib.fl_attention_prefill_plan(T, pos0, 24, 4, 256, buf, 1024)
    bins = 64
    w = _plan_weights(T, pos0, 6)
    assert n == bins + 1 + len(w)
    v = list(buf[:n])
    items = v[bins + 1:]
    assert sorted(items) == list(range(len(w)))
    assert v[0] == 0 and v[bins] == len(w) and all(v[b] <= v[b + 1] for b in range(bins))
    loads = []
    for b in range(bins):
        mine = [w[t] for t in items[v[b]:v[b + 1]]]
        assert mine == sorted(mine, reverse=True)
        loads.append(sum(mine))
    bound = max(sum(w) / bins, max(w))
    assert max(loads) <= 1.04 * bound, (max(loads), bound)


def test_prefill_plan_falls_back_to_the_tile_grid(fl):
    """No plan (a grid of row tiles x kv heads) where the kernel does not run
    (short prompts, the KV-split chunk), where the row tiles do not outnumber
    the bins, where the kv heads do not divide the 8 XCDs, or where the plan
    would pass 2 KiB of kernel arguments."""
    lib = fl._lib.lib()
    assert lib.fl_attention_prefill_plan(2048, 0, 24, 4, 256, None, 0) == 0
    assert lib.fl_attention_prefill_plan(1024, 98000, 24, 4, 256, None, 0) == 0
    assert lib.fl_attention_prefill_plan(65536, 0, 24, 4, 256, None, 0) == 0
    assert lib.fl_attention_prefill_plan(8192, 0, 24, 3, 256, None, 0) == 0
    assert lib.fl_attention_prefill_plan(8192, 0, 24, 4, 250, None, 0) == 0
    assert lib.fl_attention_prefill_plan(8192, 0, 24, 4, 256, None, 0) == 64 + 1 + 192


def test_integration_stub_matches_the_binding(fl):
    """The ctypes stub INTEGRATION.md gives a maintainer for the reference
    runtime declares the same argument lists as the package's own binding
    (the one every test calls through), entry point by entry point."""
    import ctypes
    text = (REPO / "INTEGRATION.md").read_text()
    block = text.split("```python", 1)[1].split("```", 1)[0]
    sigs_src = block.split("_SIGS = ", 1)[1]
    depth, end = 0, 0
    for n, ch in enumerate(sigs_src):
        depth += ch == "{"
        depth -= ch == "}"
        if depth == 0 and ch == "}":
            end = n + 1
            break
    names = {"_P": ctypes.c_void_p, "_I": ctypes.c_int, "_F": ctypes.c_float,
             "_LL": ctypes.c_longlong, "_SZ": ctypes.c_size_t,
             "_PP": ctypes.POINTER(ctypes.c_void_p), "_IP": ctypes.POINTER(ctypes.c_int)}
    stub = eval(sigs_src[:end], {"__builtins__": {}}, names)
    table = fl._lib.SIGNATURES
    assert len(stub) >= 25
    for name, args in stub.items():
        assert name in table, name
        assert list(args) == list(table[name][1]), name
    # the size queries the stub binds by hand
    for name, n_args in (("fl_attn_decode_work_bytes", 5), ("fl_gdn_chunked_work_bytes", 5),
                         ("fl_attention_prefill_work_bytes", 4),
                         ("fl_attention_prefill_q8_stage_bytes", 5)):
        assert name in block
        assert table[name] == (ctypes.c_size_t, [ctypes.c_int] * n_args), name
