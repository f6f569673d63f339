"""Host-side binding of the gfx950 attention forward (``libfav4_bshd.so``).

Mirrors the reference harness's ctypes binding, ``benchmarks/bshd.py:18-20``
(``Args``) and ``:56-74`` (``Runner.call``): the same argument structure, the
same argument checks, the stream taken from torch's current stream, the scale
1/sqrt(128) by default, and a ``RuntimeError`` carrying the HIP status when the
C ABI returns non-zero.  The library is the product; this module only moves
pointers.  There is no fallback: if the library is missing, loading raises.
"""
from __future__ import annotations

import ctypes as C
import math
import os
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
LIB_PATH = ROOT / "build" / "libfav4_bshd.so"
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
D = 128

HIPCC_FLAGS = [
    "-O3", "-std=c++17", "--offload-arch=gfx950", "-fPIC", "-shared", "-fvisibility=hidden",
    f"-I{INCLUDE}", f"-I{CSRC}",
    "-fgpu-flush-denormals-to-zero",
    # keep the compiler from emitting packed-FP32 VALU ops (v_pk_fma_f32 & co.)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # per-kernel VGPR / AGPR / SGPR counts, spills, LDS and occupancy, as
    # compiler remarks (the reference's scripts/build.sh:14-17 keeps the same)
    "-Rpass-analysis=kernel-resource-usage",
]
KAT_LIB_PATH = ROOT / "build" / "libfav4_loader_kat.so"
CEILING_LIB_PATH = ROOT / "build" / "libfav4_mfma_ceiling.so"
RESOURCE_LOG = ROOT / "build" / "resource-usage.txt"
MANIFEST = ROOT / "build" / "build-manifest.json"

class Args(C.Structure):
    """``struct Fav4Args`` (include/fav4_bshd.h): 5 pointers, 4 ints, 1 float."""
    _fields_ = [(n, C.c_void_p) for n in ("q", "k", "v", "o", "lse")] + [
        (n, C.c_int) for n in ("batch", "heads", "sq", "sk")] + [("scale", C.c_float)]


class VarlenArgs(C.Structure):
    """``struct Fav4VarlenArgs`` (include/fav4_bshd.h): 7 pointers, 7 ints, 1 float."""
    _fields_ = [(n, C.c_void_p) for n in ("q", "k", "v", "o", "lse", "cu_seqlens_q", "cu_seqlens_k")] + [
        (n, C.c_int) for n in ("batch", "heads", "kv_heads", "max_seqlen_q", "max_seqlen_k", "total_q",
                               "total_k")] + [("scale", C.c_float)]


class PagedArgs(C.Structure):
    """``struct Fav4PagedArgs`` (include/fav4_bshd.h): 8 pointers, 10 ints, 1 float."""
    _fields_ = [(n, C.c_void_p) for n in ("q", "k_cache", "v_cache", "o", "lse", "cu_seqlens_q", "seqlens_k",
                                          "block_table")] + [
        (n, C.c_int) for n in ("batch", "heads", "kv_heads", "max_seqlen_q", "max_seqlen_k", "total_q", "total_k",
                               "num_pages", "page_size", "max_pages_per_seq")] + [("scale", C.c_float)]


class Strides(C.Structure):
    """``struct Fav4Strides`` (include/fav4_bshd.h): element strides of a [B, S, H, 128] view."""
    _fields_ = [(n, C.c_longlong) for n in ("batch", "seq", "head")]


def parse_resource_usage(text: str) -> dict:
    """Per-kernel fields of hipcc's kernel-resource-usage remarks."""
    table, name = {}, None
    for line in text.splitlines():
        if "remark:" not in line or "kernel-resource-usage" not in line:
            continue
        body = line.split("remark:", 1)[1].rsplit("[-Rpass-analysis", 1)[0].strip()
        key, _, val = body.partition(":")
        key, val = key.strip(), val.strip()
        if key == "Function Name":
            name = val
            table[name] = {}
        elif name is not None:
            table[name][key] = int(val) if val.lstrip("-").isdigit() else val
    return table


def build_library(out: Path = LIB_PATH, verbose: bool = False) -> Path:
    """Compile ``csrc/bshd.hip`` for gfx950 into ``build/libfav4_bshd.so``, the
    loader probe ``csrc/loader_kat.hip`` into ``build/libfav4_loader_kat.so``
    (a test library) and the MFMA-only probe ``csrc/mfma_ceiling.hip`` into
    ``build/libfav4_mfma_ceiling.so`` (a measurement library, read by
    ``bench.py --mfma-ceiling``), keep the compiler's kernel-resource-usage remarks in
    ``build/resource-usage.txt`` and write ``build/build-manifest.json``
    (toolchain, flags, source and library sha256, per-kernel resources)."""
    import hashlib
    import json
    import platform
    import time
    out.parent.mkdir(parents=True, exist_ok=True)
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    jobs = {out: CSRC / "bshd.hip", KAT_LIB_PATH: CSRC / "loader_kat.hip",
            CEILING_LIB_PATH: CSRC / "mfma_ceiling.hip"}
    procs = {}
    for lib, src in jobs.items():
        tmp = lib.with_suffix(".so.tmp")
        procs[lib] = (tmp, subprocess.Popen([hipcc, *HIPCC_FLAGS, str(src), "-o", str(tmp)],
                                            stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True))
    remarks = []
    for lib, (tmp, proc) in procs.items():
        _, err = proc.communicate()
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc failed ({proc.returncode}) on {jobs[lib].name}:\n{err[-4000:]}")
        if verbose and err:
            print(err)
        remarks.append(err)
        os.replace(tmp, lib)
    text = "\n".join(remarks)
    RESOURCE_LOG.write_text(text)
    sha = lambda p: hashlib.sha256(Path(p).read_bytes()).hexdigest()
    version = subprocess.run([hipcc, "--version"], capture_output=True, text=True).stdout
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.hpp")) + [INCLUDE / "fav4_bshd.h"]
    manifest = {
        "built_at": time.strftime("%Y-%m-%dT%H:%M:%SZ", time.gmtime()),
        "host": platform.node(),
        "hipcc": hipcc, "hipcc_version": [ln for ln in version.splitlines() if ln.strip()][:3],
        "flags": HIPCC_FLAGS,
        "sources": {str(p.relative_to(ROOT)): sha(p) for p in sources},
        "libraries": {lib.name: {"sha256": sha(lib), "bytes": lib.stat().st_size, "source": jobs[lib].name}
                      for lib in jobs},
        "kernel_resources": parse_resource_usage(text),
    }
    MANIFEST.write_text(json.dumps(manifest, indent=1))
    return out


_LIB = None


def load_library(path: Path = LIB_PATH) -> C.CDLL:
    """Load the built library (raises OSError if it is missing).

    PyTorch-ROCm wheels bundle their own HIP and HSA runtimes. Torch is
    therefore imported first when it is installed. The library's
    libamdhip64.so.7 dependency then binds to the runtime already in the
    process, and torch's streams and the library share one runtime.
    Loaded the other way round, the process holds two HIP runtimes, and
    the library's launches fail with hipErrorNoDevice (100)."""
    global _LIB
    if _LIB is None or Path(_LIB._name) != Path(path):
        if not Path(path).exists():
            raise OSError(f"{path} not built; run __graft_entry__.build() first")
        try:
            import torch  # noqa: F401  (binds the library to torch's HIP runtime)
        except ImportError:
            pass
        lib = C.CDLL(str(path))
        lib.fav4_bshd_forward.argtypes = [C.POINTER(Args), C.c_int, C.c_int, C.c_void_p]
        lib.fav4_bshd_forward.restype = C.c_int
        lib.fav4_bshd_select_config.argtypes = [C.POINTER(Args)]
        lib.fav4_bshd_select_config.restype = C.c_int
        lib.fav4_bshd_select_config_masked.argtypes = [C.POINTER(Args), C.c_int]
        lib.fav4_bshd_select_config_masked.restype = C.c_int
        lib.fav4_bshd_forward_splitkv.argtypes = [C.POINTER(Args), C.c_int, C.c_int, C.c_void_p, C.c_size_t,
                                                  C.c_void_p]
        lib.fav4_bshd_forward_splitkv.restype = C.c_int
        lib.fav4_bshd_splitkv_workspace_size.argtypes = [C.POINTER(Args), C.c_int, C.c_int]
        lib.fav4_bshd_splitkv_workspace_size.restype = C.c_longlong
        lib.fav4_bshd_splitkv_select.argtypes = [C.POINTER(Args), C.c_int]
        lib.fav4_bshd_splitkv_select.restype = C.c_int
        lib.fav4_bshd_forward_splitkv_gqa.argtypes = [C.POINTER(Args), C.c_int, C.c_int, C.c_int, C.c_void_p,
                                                      C.c_size_t, C.c_void_p]
        lib.fav4_bshd_forward_splitkv_gqa.restype = C.c_int
        lib.fav4_bshd_splitkv_gqa_workspace_size.argtypes = [C.POINTER(Args), C.c_int, C.c_int, C.c_int]
        lib.fav4_bshd_splitkv_gqa_workspace_size.restype = C.c_longlong
        lib.fav4_bshd_splitkv_gqa_select.argtypes = [C.POINTER(Args), C.c_int, C.c_int]
        lib.fav4_bshd_splitkv_gqa_select.restype = C.c_int
        lib.fav4_bshd_forward_splitkv_gqa_noalloc.argtypes = [C.POINTER(Args), C.c_int, C.c_int, C.c_int,
                                                              C.c_void_p]
        lib.fav4_bshd_forward_splitkv_gqa_noalloc.restype = C.c_int
        lib.fav4_bshd_forward_gqa.argtypes = [C.POINTER(Args), C.c_int, C.c_int, C.c_int, C.c_void_p]
        lib.fav4_bshd_forward_gqa.restype = C.c_int
        lib.fav4_bshd_forward_strided.argtypes = [C.POINTER(Args), C.c_int] + [C.POINTER(Strides)] * 4 + [
            C.c_int, C.c_int, C.c_void_p]
        lib.fav4_bshd_forward_strided.restype = C.c_int
        lib.fav4_bshd_forward_varlen.argtypes = [C.POINTER(VarlenArgs), C.c_int, C.c_void_p]
        lib.fav4_bshd_forward_varlen.restype = C.c_int
        lib.fav4_bshd_forward_splitkv_varlen.argtypes = [C.POINTER(VarlenArgs), C.c_int, C.c_int, C.c_void_p,
                                                         C.c_size_t, C.c_void_p]
        lib.fav4_bshd_forward_splitkv_varlen.restype = C.c_int
        lib.fav4_bshd_splitkv_varlen_workspace_size.argtypes = [C.POINTER(VarlenArgs), C.c_int, C.c_int]
        lib.fav4_bshd_splitkv_varlen_workspace_size.restype = C.c_longlong
        lib.fav4_bshd_splitkv_varlen_select.argtypes = [C.POINTER(VarlenArgs), C.c_int]
        lib.fav4_bshd_splitkv_varlen_select.restype = C.c_int
        lib.fav4_bshd_forward_splitkv_paged.argtypes = [C.POINTER(PagedArgs), C.c_int, C.c_int, C.c_void_p,
                                                        C.c_size_t, C.c_void_p]
        lib.fav4_bshd_forward_splitkv_paged.restype = C.c_int
        lib.fav4_bshd_splitkv_paged_workspace_size.argtypes = [C.POINTER(PagedArgs), C.c_int, C.c_int]
        lib.fav4_bshd_splitkv_paged_workspace_size.restype = C.c_longlong
        lib.fav4_bshd_splitkv_paged_select.argtypes = [C.POINTER(PagedArgs), C.c_int]
        lib.fav4_bshd_splitkv_paged_select.restype = C.c_int
        _LIB = lib
    return _LIB


class Runner:
    """ctypes runner with the reference harness's call signature (bshd.py:56-74)."""

    def __init__(self, path: Path = LIB_PATH):
        self.hip = load_library(path)

    def args(self, q, k, v, o, lse, scale=None, kv_heads=None) -> Args:
        import torch
        assert all(x.dtype == torch.bfloat16 and x.is_cuda and x.is_contiguous() for x in (q, k, v, o))
        b, sq, h, d = q.shape
        kvh = h if kv_heads is None else kv_heads
        assert d == D and k.shape == v.shape and k.shape[0] == b and tuple(k.shape[2:]) == (kvh, d)
        assert o.shape == q.shape
        assert lse is None or (tuple(lse.shape) == (b, h, sq) and lse.is_contiguous()
                               and lse.dtype == torch.float32)
        return Args(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                    lse.data_ptr() if lse is not None else None,
                    b, h, sq, k.shape[1], 1 / math.sqrt(d) if scale is None else scale)

    def call(self, q, k, v, o, lse, causal, config=0, scale=None, stream=None):
        import torch
        a = self.args(q, k, v, o, lse, scale)
        if stream is None:
            stream = torch.cuda.current_stream().cuda_stream
        status = self.hip.fav4_bshd_forward(C.byref(a), int(causal), int(config), stream)
        if status:
            raise RuntimeError(f"config {config}: HIP status {status}")

    def call_gqa(self, q, k, v, o, lse, causal, config=0, scale=None, stream=None):
        """fav4_bshd_forward_gqa: K/V heads = k.shape[2] (must divide q's heads)."""
        import torch
        a = self.args(q, k, v, o, lse, scale, kv_heads=k.shape[2])
        if stream is None:
            stream = torch.cuda.current_stream().cuda_stream
        status = self.hip.fav4_bshd_forward_gqa(C.byref(a), int(k.shape[2]), int(causal), int(config), stream)
        if status:
            raise RuntimeError(f"gqa config {config}: HIP status {status}")

    def select_config(self, q, k, causal=None) -> int:
        """Config ID that config 0 resolves to: the reference's dense query
        when `causal` is None, else fav4_bshd_select_config_masked."""
        b, sq, h, _ = q.shape
        a = Args(None, None, None, None, None, b, h, sq, k.shape[1], 1 / math.sqrt(D))
        if causal is None:
            return self.hip.fav4_bshd_select_config(C.byref(a))
        return self.hip.fav4_bshd_select_config_masked(C.byref(a), int(causal))

    # ---- split-KV (fav4_bshd_forward_splitkv; no reference counterpart) ----
    @staticmethod
    def shape_args(batch, heads, sq, sk) -> Args:
        return Args(None, None, None, None, None, batch, heads, sq, sk, 1 / math.sqrt(D))

    def splitkv_select(self, batch, heads, sq, sk, causal, kv_heads=None) -> int:
        a = self.shape_args(batch, heads, sq, sk)
        if kv_heads is None:
            return self.hip.fav4_bshd_splitkv_select(C.byref(a), int(causal))
        return self.hip.fav4_bshd_splitkv_gqa_select(C.byref(a), int(kv_heads), int(causal))

    def splitkv_workspace_size(self, batch, heads, sq, sk, causal, splits=0, kv_heads=None) -> int:
        a = self.shape_args(batch, heads, sq, sk)
        if kv_heads is None:
            return self.hip.fav4_bshd_splitkv_workspace_size(C.byref(a), int(causal), int(splits))
        return self.hip.fav4_bshd_splitkv_gqa_workspace_size(C.byref(a), int(kv_heads), int(causal), int(splits))

    def call_splitkv(self, q, k, v, o, lse, causal, splits=0, workspace=None, scale=None, stream=None):
        """Split-KV forward; K/V heads = k.shape[2] (fewer than q's: the GQA
        entry point).  `workspace` is a CUDA tensor (any dtype, 256-byte
        aligned); None allocates one of the required size here (the library
        never allocates)."""
        import torch
        kvh = k.shape[2]
        gqa = kvh != q.shape[2]
        a = self.args(q, k, v, o, lse, scale, kv_heads=kvh)
        if workspace is None:
            if gqa:
                need = self.hip.fav4_bshd_splitkv_gqa_workspace_size(C.byref(a), int(kvh), int(causal), int(splits))
            else:
                need = self.hip.fav4_bshd_splitkv_workspace_size(C.byref(a), int(causal), int(splits))
            if need < 0:
                raise RuntimeError(f"splits {splits}: arguments rejected")
            workspace = torch.empty(max(need, 1), device=q.device, dtype=torch.uint8)
        nbytes = workspace.numel() * workspace.element_size()
        if stream is None:
            stream = torch.cuda.current_stream().cuda_stream
        if gqa:
            status = self.hip.fav4_bshd_forward_splitkv_gqa(C.byref(a), int(kvh), int(causal), int(splits),
                                                             workspace.data_ptr(), nbytes, stream)
        else:
            status = self.hip.fav4_bshd_forward_splitkv(C.byref(a), int(causal), int(splits), workspace.data_ptr(),
                                                         nbytes, stream)
        if status:
            raise RuntimeError(f"splitkv splits {splits}: HIP status {status}")
        return workspace

    def call_splitkv_noalloc(self, q, k, v, o, lse, causal, splits=0, scale=None, stream=None):
        """fav4_bshd_forward_splitkv_gqa_noalloc: split-KV with the library's own
        64 MiB per-device partials array (no workspace); K/V heads = k.shape[2]."""
        import torch
        kvh = k.shape[2]
        a = self.args(q, k, v, o, lse, scale, kv_heads=kvh)
        if stream is None:
            stream = torch.cuda.current_stream().cuda_stream
        status = self.hip.fav4_bshd_forward_splitkv_gqa_noalloc(C.byref(a), int(kvh), int(causal), int(splits),
                                                                 stream)
        if status:
            raise RuntimeError(f"splitkv noalloc splits {splits}: HIP status {status}")

    # ---- arbitrary strides (fav4_bshd_forward_strided; no reference counterpart) ----
    def call_strided(self, q, k, v, o, lse, causal, config=0, scale=None, stream=None):
        """q/o: [B, Sq, H, 128] and k/v: [B, Sk, KVH, 128] views with any strides whose last
        dimension is contiguous (e.g. ``x_bhsd.transpose(1, 2)``, ``qkv[:, :, 0]``);
        lse: FP32 [B, H, Sq] contiguous or None."""
        import torch
        for x in (q, k, v, o):
            assert x.dtype == torch.bfloat16 and x.is_cuda and x.dim() == 4 and x.shape[3] == D and x.stride(3) == 1
        b, sq, h, _ = q.shape
        assert o.shape == q.shape and k.shape == v.shape and k.shape[0] == b
        assert lse is None or (tuple(lse.shape) == (b, h, sq) and lse.is_contiguous() and lse.dtype == torch.float32)
        a = Args(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                 lse.data_ptr() if lse is not None else None, b, h, sq, k.shape[1],
                 1 / math.sqrt(D) if scale is None else scale)
        st = [Strides(x.stride(0), x.stride(1), x.stride(2)) for x in (q, k, v, o)]
        if stream is None:
            stream = torch.cuda.current_stream().cuda_stream
        status = self.hip.fav4_bshd_forward_strided(C.byref(a), int(k.shape[2]), *[C.byref(x) for x in st],
                                                    int(causal), int(config), stream)
        if status:
            raise RuntimeError(f"strided config {config}: HIP status {status}")

    # ---- packed variable-length sequences (fav4_bshd_forward_varlen; no reference counterpart) ----
    def varlen_args(self, q, k, v, o, lse, cu_q, cu_k, max_q, max_k, scale=None) -> VarlenArgs:
        """q/o: [total_q, heads, 128]; k/v: [total_k, kv_heads, 128] (BF16, contiguous);
        cu_q/cu_k: int32 [batch+1] on the device; lse: FP32 [heads, total_q] or None."""
        import torch
        assert all(x.dtype == torch.bfloat16 and x.is_cuda and x.is_contiguous() for x in (q, k, v, o))
        assert q.dim() == 3 and q.shape[2] == D and o.shape == q.shape and k.shape == v.shape and k.dim() == 3
        assert all(c.dtype == torch.int32 and c.is_cuda and c.is_contiguous() and c.dim() == 1 for c in (cu_q, cu_k))
        assert cu_q.numel() == cu_k.numel() >= 2
        tq, h, _ = q.shape
        assert lse is None or (tuple(lse.shape) == (h, tq) and lse.is_contiguous() and lse.dtype == torch.float32)
        return VarlenArgs(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                          lse.data_ptr() if lse is not None else None, cu_q.data_ptr(), cu_k.data_ptr(),
                          cu_q.numel() - 1, h, k.shape[1], int(max_q), int(max_k), tq, k.shape[0],
                          1 / math.sqrt(D) if scale is None else scale)

    def call_varlen(self, q, k, v, o, lse, cu_q, cu_k, max_q, max_k, causal, scale=None, stream=None):
        import torch
        a = self.varlen_args(q, k, v, o, lse, cu_q, cu_k, max_q, max_k, scale)
        if stream is None:
            stream = torch.cuda.current_stream().cuda_stream
        status = self.hip.fav4_bshd_forward_varlen(C.byref(a), int(causal), stream)
        if status:
            raise RuntimeError(f"varlen: HIP status {status}")

    # ---- split-KV of packed batches (fav4_bshd_forward_splitkv_varlen; no reference counterpart) ----
    @staticmethod
    def varlen_shape_args(batch, heads, kv_heads, max_q, max_k, total_q, total_k) -> VarlenArgs:
        """Shape-only arguments for the select / workspace queries (no buffers)."""
        return VarlenArgs(None, None, None, None, None, None, None, batch, heads, kv_heads, max_q, max_k,
                          total_q, total_k, 1 / math.sqrt(D))

    def splitkv_varlen_select(self, batch, heads, kv_heads, max_q, max_k, total_q, total_k, causal) -> int:
        a = self.varlen_shape_args(batch, heads, kv_heads, max_q, max_k, total_q, total_k)
        return self.hip.fav4_bshd_splitkv_varlen_select(C.byref(a), int(causal))

    def splitkv_varlen_workspace_size(self, batch, heads, kv_heads, max_q, max_k, total_q, total_k, causal,
                                      splits=0) -> int:
        a = self.varlen_shape_args(batch, heads, kv_heads, max_q, max_k, total_q, total_k)
        return self.hip.fav4_bshd_splitkv_varlen_workspace_size(C.byref(a), int(causal), int(splits))

    def call_splitkv_varlen(self, q, k, v, o, lse, cu_q, cu_k, max_q, max_k, causal, splits=0, workspace=None,
                            scale=None, stream=None):
        """Split-KV over packed sequences; tensors as for call_varlen.  `workspace`
        as for call_splitkv (None: allocated here)."""
        import torch
        a = self.varlen_args(q, k, v, o, lse, cu_q, cu_k, max_q, max_k, scale)
        if workspace is None:
            need = self.hip.fav4_bshd_splitkv_varlen_workspace_size(C.byref(a), int(causal), int(splits))
            if need < 0:
                raise RuntimeError(f"splitkv varlen splits {splits}: arguments rejected")
            workspace = torch.empty(max(need, 1), device=q.device, dtype=torch.uint8)
        nbytes = workspace.numel() * workspace.element_size()
        if stream is None:
            stream = torch.cuda.current_stream().cuda_stream
        status = self.hip.fav4_bshd_forward_splitkv_varlen(C.byref(a), int(causal), int(splits),
                                                            workspace.data_ptr(), nbytes, stream)
        if status:
            raise RuntimeError(f"splitkv varlen splits {splits}: HIP status {status}")
        return workspace


    # ---- split-KV decode over paged K/V caches (no reference counterpart) ----
    def paged_args(self, q, k_cache, v_cache, o, lse, cu_q, seqlens_k, block_table, max_q, max_k, total_k=None,
                   scale=None) -> PagedArgs:
        """q/o: [total_q, heads, 128]; k_cache/v_cache: [num_pages, page_size, kv_heads, 128] (BF16,
        contiguous); cu_q: int32 [batch+1]; seqlens_k: int32 [batch]; block_table: int32
        [batch, max_pages_per_seq] (device tensors); lse: FP32 [heads, total_q] or None.  total_k
        (cached keys over the batch) only steers Auto; None passes max_k * batch."""
        import torch
        assert all(x.dtype == torch.bfloat16 and x.is_cuda and x.is_contiguous() for x in (q, k_cache, v_cache, o))
        assert q.dim() == 3 and q.shape[2] == D and o.shape == q.shape
        assert k_cache.dim() == 4 and k_cache.shape == v_cache.shape and k_cache.shape[3] == D
        assert all(c.dtype == torch.int32 and c.is_cuda and c.is_contiguous() for c in (cu_q, seqlens_k, block_table))
        assert block_table.dim() == 2 and cu_q.numel() == seqlens_k.numel() + 1 == block_table.shape[0] + 1
        tq, h, _ = q.shape
        assert lse is None or (tuple(lse.shape) == (h, tq) and lse.is_contiguous() and lse.dtype == torch.float32)
        b = seqlens_k.numel()
        return PagedArgs(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), o.data_ptr(),
                         lse.data_ptr() if lse is not None else None, cu_q.data_ptr(), seqlens_k.data_ptr(),
                         block_table.data_ptr(), b, h, k_cache.shape[2], int(max_q), int(max_k), tq,
                         int(max_k) * b if total_k is None else int(total_k), k_cache.shape[0], k_cache.shape[1],
                         block_table.shape[1], 1 / math.sqrt(D) if scale is None else scale)

    @staticmethod
    def paged_shape_args(batch, heads, kv_heads, max_q, max_k, total_q, total_k, page_size, max_pages,
                         num_pages) -> PagedArgs:
        """Shape-only arguments for the select / workspace queries (no buffers)."""
        return PagedArgs(None, None, None, None, None, None, None, None, batch, heads, kv_heads, max_q, max_k, total_q,
                         total_k, num_pages, page_size, max_pages, 1 / math.sqrt(D))

    def splitkv_paged_select(self, batch, heads, kv_heads, max_q, max_k, total_q, total_k, page_size, max_pages,
                             num_pages, causal=0) -> int:
        """Auto chunk count for call_splitkv_paged with the same mask (0 dense, 2 bottom-right)."""
        a = self.paged_shape_args(batch, heads, kv_heads, max_q, max_k, total_q, total_k, page_size, max_pages,
                                  num_pages)
        return self.hip.fav4_bshd_splitkv_paged_select(C.byref(a), int(causal))

    def splitkv_paged_workspace_size(self, batch, heads, kv_heads, max_q, max_k, total_q, total_k, page_size,
                                     max_pages, num_pages, splits=0, causal=0) -> int:
        """Workspace bytes of call_splitkv_paged with the same mask (0 dense, 2 bottom-right):
        the chunk plan, and so the size, depends on it."""
        a = self.paged_shape_args(batch, heads, kv_heads, max_q, max_k, total_q, total_k, page_size, max_pages,
                                  num_pages)
        return self.hip.fav4_bshd_splitkv_paged_workspace_size(C.byref(a), int(causal), int(splits))

    def call_splitkv_paged(self, q, k_cache, v_cache, o, lse, cu_q, seqlens_k, block_table, max_q, max_k,
                           splits=0, workspace=None, total_k=None, scale=None, stream=None, causal=0):
        """Decode over paged caches (causal 0 = dense, 2 = bottom-right); `workspace` as for
        call_splitkv (None: allocated here)."""
        import torch
        a = self.paged_args(q, k_cache, v_cache, o, lse, cu_q, seqlens_k, block_table, max_q, max_k, total_k, scale)
        if workspace is None:
            need = self.hip.fav4_bshd_splitkv_paged_workspace_size(C.byref(a), int(causal), int(splits))
            if need < 0:
                raise RuntimeError(f"splitkv paged splits {splits}: arguments rejected")
            workspace = torch.empty(max(need, 1), device=q.device, dtype=torch.uint8)
        nbytes = workspace.numel() * workspace.element_size()
        if stream is None:
            stream = torch.cuda.current_stream().cuda_stream
        status = self.hip.fav4_bshd_forward_splitkv_paged(C.byref(a), int(causal), int(splits), workspace.data_ptr(),
                                                           nbytes, stream)
        if status:
            raise RuntimeError(f"splitkv paged splits {splits}: HIP status {status}")
        return workspace


def forward(q, k, v, causal=False, with_lse=False, config=0, scale=None):
    """Allocate O (and LSE) and run the forward; returns (o, lse or None)."""
    import torch
    o = torch.empty_like(q)
    lse = (torch.empty((q.shape[0], q.shape[2], q.shape[1]), device=q.device, dtype=torch.float32)
           if with_lse else None)
    Runner().call(q, k, v, o, lse, causal, config, scale)
    return o, lse
