"""C-ABI checks that need no GPU: the library loads, exports exactly what the
header declares (with the legacy prototypes of crates/rocm-backend/src/ops.rs:315-332
and :554-594),
and rejects bad arguments on the host before any HIP call."""
import ctypes
import re
import subprocess

from physllm_amd import capi

LEGACY = ["launch_moe_router", "launch_moe_expert_silu", "launch_moe_expert_down",
          "launch_moe_combine", "launch_mxfp4_dequant", "launch_rms_norm", "launch_residual_add"]


def test_library_exports_every_header_symbol():
    syms = capi.header_symbols()
    assert set(LEGACY) <= set(syms)
    out = subprocess.run(["nm", "-D", "--defined-only", capi.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    missing = [s for s in syms if s not in exported]
    assert not missing, missing
    # nothing beyond the header leaks out of the library
    extra = sorted(s for s in exported if s not in syms)
    assert not extra, extra
    L = capi.lib()
    for s in syms:
        assert getattr(L, s) is not None


def test_legacy_prototypes_match_rust_ffi():
    """Parameter counts/types of the legacy launchers equal the Rust extern block."""
    hdr = open(capi.HEADER_PATH).read()
    expect = {
        "launch_moe_router": ["const void*", "const void*", "void*", "void*", "int", "int", "int", "int", "void*"],
        "launch_moe_expert_silu": ["const void*", "const void*", "const void*", "void*", "int", "int", "void*"],
        "launch_moe_expert_down": ["const void*", "const void*", "void*", "int", "int", "void*"],
        "launch_moe_combine": ["const void*", "const void*", "void*", "int", "int", "void*"],
        "launch_mxfp4_dequant": ["const void*", "const void*", "void*", "int", "int", "void*"],
        # ops.rs:315-319 and :329-332
        "launch_rms_norm": ["const void*", "const void*", "void*", "int", "int", "float", "void*"],
        "launch_residual_add": ["void*", "const void*", "int", "void*"],
    }
    for name, types in expect.items():
        m = re.search(r"void\s+" + name + r"\s*\(([^)]*)\)", hdr)
        assert m, name
        params = [re.sub(r"\s+", " ", p.strip()) for p in m.group(1).split(",")]
        got = [re.sub(r"\s*\w+$", "", p).replace(" *", "*") for p in params]
        assert got == types, (name, got)


def test_workspace_query_and_validation_without_gpu():
    L = capi.lib()
    cfg = capi.MoEConfig(2880, 2880, 32, 4, 1.702, 7.0)
    n1 = L.physllm_moe_workspace_bytes(ctypes.byref(cfg), 1)
    n64 = L.physllm_moe_workspace_bytes(ctypes.byref(cfg), 64)
    assert n1 > 0 and n64 > n1
    # y (fp32 [B*k, H]) and h (bf16 [B*k, I]) dominate
    assert n64 >= 64 * 4 * (2880 * 4 + 2880 * 2)
    bad = capi.MoEConfig(2880, 2880, 32, 33, 1.702, 7.0)       # top_k > num_experts
    assert L.physllm_moe_workspace_bytes(ctypes.byref(bad), 1) == 0
    assert L.physllm_moe_last_error() == capi.PHYSLLM_MOE_EINVAL
    bad = capi.MoEConfig(2881, 2880, 32, 4, 1.702, 7.0)        # hidden not a multiple of 32
    assert L.physllm_moe_workspace_bytes(ctypes.byref(bad), 1) == 0
    assert b"multiple of 32" in L.physllm_moe_last_error_message()
    assert L.physllm_moe_workspace_bytes(ctypes.byref(cfg), 1) > 0
    assert L.physllm_moe_last_error() == 0


def test_layer_rejects_bad_arguments_on_host():
    L = capi.lib()
    cfg = capi.MoEConfig(2880, 2880, 32, 4, 1.702, 7.0)
    w = capi.MoEWeights()
    rc = L.physllm_moe_layer_forward(ctypes.byref(cfg), ctypes.byref(w), None, -1, None, None, None, None, 0, None)
    assert rc == capi.PHYSLLM_MOE_EINVAL
    rc = L.physllm_moe_layer_forward(ctypes.byref(cfg), ctypes.byref(w), None, 0, None, None, None, None, 0, None)
    assert rc == capi.PHYSLLM_MOE_OK                                # empty batch is a no-op
    rc = L.physllm_moe_layer_forward(ctypes.byref(cfg), ctypes.byref(w), None, 4, None, None, None, None, 0, None)
    assert rc == capi.PHYSLLM_MOE_EINVAL and b"null" in L.physllm_moe_last_error_message()
    fake = ctypes.c_void_p(0x1000)
    w2 = capi.MoEWeights(fake, None, fake, fake, None, fake, fake, None)
    rc = L.physllm_moe_layer_forward(ctypes.byref(cfg), ctypes.byref(w2), fake, 4, fake, None, None, fake, 16, None)
    assert rc == capi.PHYSLLM_MOE_EWORKSPACE
    rc = L.physllm_moe_route_topk(fake, fake, None, 4, 2880, 32, 0, fake, fake, None)
    assert rc == capi.PHYSLLM_MOE_EINVAL
    rc = L.physllm_moe_route_topk(fake, fake, None, 4, 2880, 2048, 4, fake, fake, None)
    assert rc == capi.PHYSLLM_MOE_EINVAL and b"1024" in L.physllm_moe_last_error_message()
    rc = L.physllm_moe_mxfp4_dequant(fake, fake, fake, -5, None)
    assert rc == capi.PHYSLLM_MOE_EINVAL
    rc = L.physllm_moe_mxfp4_dequant(fake, fake, fake, 0, None)
    assert rc == capi.PHYSLLM_MOE_OK
    # legacy void launchers report through the last-error channel
    L.launch_moe_router(fake, fake, fake, fake, 1, 2880, 32, 40, None)
    assert L.physllm_moe_last_error() == capi.PHYSLLM_MOE_EINVAL
    L.launch_mxfp4_dequant(fake, fake, fake, 64, 0, None)
    assert L.physllm_moe_last_error() == capi.PHYSLLM_MOE_EINVAL
    L.launch_moe_combine(None, None, None, 2880, 4, None)
    assert L.physllm_moe_last_error() == capi.PHYSLLM_MOE_EINVAL


def test_block_workspace_and_validation_without_gpu():
    """The block entry (moe.rs:238-313) needs the layer's workspace plus B*H bf16
    for the normalised activations, and checks its arguments before any launch."""
    L = capi.lib()
    cfg = capi.MoEConfig(2880, 2880, 32, 4, 1.702, 7.0)
    for B in (1, 7, 64, 4096):
        lay = L.physllm_moe_workspace_bytes(ctypes.byref(cfg), B)
        blk = L.physllm_moe_block_workspace_bytes(ctypes.byref(cfg), B)
        assert blk == lay + ((B * 2880 * 2 + 255) // 256) * 256
    bad = capi.MoEConfig(2880, 2880, 32, 0, 1.702, 7.0)
    assert L.physllm_moe_block_workspace_bytes(ctypes.byref(bad), 1) == 0
    assert L.physllm_moe_last_error() == capi.PHYSLLM_MOE_EINVAL
    fake = ctypes.c_void_p(0x1000)
    w = capi.MoEWeights(fake, None, fake, fake, None, fake, fake, None)
    args = lambda x, nw, B, out, ws, n: (ctypes.byref(cfg), ctypes.byref(w), x, nw, 1e-5, B, out, None, None,
                                         ws, n, None)
    assert L.physllm_moe_block_forward(*args(None, None, 0, None, None, 0)) == capi.PHYSLLM_MOE_OK
    assert L.physllm_moe_block_forward(*args(fake, fake, -1, fake, fake, 1 << 30)) == capi.PHYSLLM_MOE_EINVAL
    assert L.physllm_moe_block_forward(*args(fake, None, 2, fake, fake, 1 << 30)) == capi.PHYSLLM_MOE_EINVAL
    assert b"norm_w" in L.physllm_moe_last_error_message()
    need = L.physllm_moe_block_workspace_bytes(ctypes.byref(cfg), 2)
    assert L.physllm_moe_block_forward(*args(fake, fake, 2, fake, fake, need - 1)) == capi.PHYSLLM_MOE_EWORKSPACE
    w0 = capi.MoEWeights()
    rc = L.physllm_moe_block_forward(ctypes.byref(cfg), ctypes.byref(w0), fake, fake, 1e-5, 2, fake, None, None,
                                     fake, need, None)
    assert rc == capi.PHYSLLM_MOE_EINVAL and b"weight" in L.physllm_moe_last_error_message()
    # legacy launchers: bad sizes and null pointers are refused, empty work is a no-op
    L.launch_rms_norm(fake, fake, fake, 1, 0, 1e-5, None)
    assert L.physllm_moe_last_error() == capi.PHYSLLM_MOE_EINVAL
    L.launch_rms_norm(fake, None, fake, 1, 2880, 1e-5, None)
    assert L.physllm_moe_last_error() == capi.PHYSLLM_MOE_EINVAL
    L.launch_rms_norm(fake, fake, fake, 0, 2880, 1e-5, None)
    assert L.physllm_moe_last_error() == 0
    L.launch_residual_add(fake, fake, -1, None)
    assert L.physllm_moe_last_error() == capi.PHYSLLM_MOE_EINVAL
    L.launch_residual_add(None, fake, 8, None)
    assert L.physllm_moe_last_error() == capi.PHYSLLM_MOE_EINVAL
    L.launch_residual_add(fake, fake, 0, None)
    assert L.physllm_moe_last_error() == 0
