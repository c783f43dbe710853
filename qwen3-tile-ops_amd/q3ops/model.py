"""Model-level binding: a device-resident PQWF blob driven through
q3_forward_chunk / q3_generate (src/main_big.cpp:145-369).

The blob lives in one torch uint8 device tensor (torch is only the allocator
and the stream provider here); the C library addresses every table by its
tools/pqwf.py offset.  Stage buffers are read back by offset, like the
reference's blob dump.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from ._lib import LM_ARGMAX, LM_LOGITS, LM_NONE, check, lib
from .layout import InitConfig, Layout, init_random_blob

__all__ = ["Model", "LM_NONE", "LM_LOGITS", "LM_ARGMAX"]


class Model:
    def __init__(self, layout: Layout, blob_host: np.ndarray | None = None,
                 init: InitConfig | None = None, device: str = "cuda",
                 stream: torch.cuda.Stream | None = None):
        self.layout = layout
        if blob_host is None:
            blob_host = init_random_blob(layout, init or InitConfig())
        self.blob = torch.empty(layout.size, dtype=torch.uint8, device=device)
        self.blob.copy_(torch.from_numpy(blob_host[:layout.size]))
        self.stream = stream or torch.cuda.current_stream()
        torch.cuda.synchronize()
        h = C.c_void_p()
        check(lib().q3_model_open(C.c_void_p(self.blob.data_ptr()), C.byref(layout.c),
                                  C.c_void_p(self.stream.cuda_stream), C.byref(h)),
              "q3_model_open")
        self.handle = h

    # -- execution ----------------------------------------------------------
    def generate(self) -> None:
        """main_big.cpp:332-369: reads CTRL from the blob, writes ids."""
        check(lib().q3_generate(self.handle), "q3_generate")

    def forward_chunk(self, pos: int, rows: int, lm_out: int = LM_NONE,
                      optimize_tail: bool = False) -> None:
        check(lib().q3_forward_chunk(self.handle, pos, rows, lm_out, int(optimize_tail)),
              "q3_forward_chunk")

    def set_page_table(self, table: np.ndarray) -> None:
        t = np.ascontiguousarray(table, dtype=np.uint16)
        check(lib().q3_model_set_page_table(self.handle, t.ctypes.data_as(C.c_void_p), t.size),
              "q3_model_set_page_table")
        self.page_table = t

    def synchronize(self) -> None:
        self.stream.synchronize()

    def decode_batch(self, ids: torch.Tensor, pos, tables, out_ids: torch.Tensor) -> None:
        """q3_decode_batch: one token for each of n independent sequences.
        ids/out_ids: int32 device tensors [n]; pos: host int32 [n]; tables:
        host uint16 [n][ld_table] (logical -> physical pages)."""
        pos = np.ascontiguousarray(pos, np.int32)
        tables = np.ascontiguousarray(tables, np.uint16)
        n = pos.shape[0]
        assert tables.ndim == 2 and tables.shape[0] == n
        assert ids.dtype == torch.int32 and ids.is_cuda and ids.numel() >= n
        assert out_ids.dtype == torch.int32 and out_ids.is_cuda and out_ids.numel() >= n
        check(lib().q3_decode_batch(self.handle, n, C.c_void_p(ids.data_ptr()),
                                    pos.ctypes.data_as(C.c_void_p),
                                    tables.ctypes.data_as(C.c_void_p), tables.shape[1],
                                    C.c_void_p(out_ids.data_ptr())), "q3_decode_batch")

    # decode kernel classes of q3_model_set_kernel_timing (include/q3ops.h)
    KERNEL_CLASSES = ("attn_decode", "gemv_qkv", "gemv_o", "gemv_gate_up", "gemv_down", "lm_head")

    def set_kernel_timing(self, enable: bool = True) -> None:
        """Brackets every launch of each decode kernel class with HIP events
        on the model's stream (a measurement aid; off by default)."""
        mask = (1 << len(self.KERNEL_CLASSES)) - 1 if enable else 0
        check(lib().q3_model_set_kernel_timing(self.handle, mask), "q3_model_set_kernel_timing")

    def kernel_times(self) -> dict:
        """{class: (total_ms, launches)} since set_kernel_timing(True)."""
        out = {}
        for i, name in enumerate(self.KERNEL_CLASSES):
            ms, n = C.c_double(0.0), C.c_uint32(0)
            check(lib().q3_model_kernel_time(self.handle, i, C.byref(ms), C.byref(n)),
                  "q3_model_kernel_time")
            out[name] = (ms.value, n.value)
        return out

    def repack(self) -> None:
        """Refresh the packed weight copy after writing new layer weights
        into the device blob (q3_model_repack)."""
        check(lib().q3_model_repack(self.handle), "q3_model_repack")

    def write(self, off: int, data: np.ndarray) -> None:
        """Host bytes into the device blob at byte offset off, ordered with
        the model's launches."""
        a = np.ascontiguousarray(data).view(np.uint8).ravel()
        with torch.cuda.stream(self.stream):
            self.blob[off:off + a.size].copy_(torch.from_numpy(a))

    def fused_status(self) -> tuple[int, int]:
        """(bit 0: a decode token's Q|K|V projection shares the attention's
        launch, bit 1: the previous layer's down projection runs in it too;
        1 if one of their bounded waits ever ran out since open, else 0).
        Synchronises the model's stream."""
        fused, gave_up = C.c_uint32(0), C.c_uint32(0)
        check(lib().q3_model_fused_status(self.handle, C.byref(fused), C.byref(gave_up)),
              "q3_model_fused_status")
        return fused.value, gave_up.value

    def close(self) -> None:
        if self.handle:
            check(lib().q3_model_close(self.handle), "q3_model_close")
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- control block / ids --------------------------------------------------
    def set_ctrl(self, n_prompt: int, n_gen: int, mode: int) -> None:
        o = self.layout.offsets
        ctrl = np.array([n_prompt, n_gen, self.layout.max_seq, mode], np.int32)
        with torch.cuda.stream(self.stream):  # ordered with the model's launches
            self.blob[o["kCTRL"]:o["kCTRL"] + 16].copy_(torch.from_numpy(ctrl.view(np.uint8)))

    def set_ids(self, ids) -> None:
        o = self.layout.offsets
        a = np.ascontiguousarray(np.asarray(ids, np.int32))
        with torch.cuda.stream(self.stream):
            self.blob[o["kIDS"]:o["kIDS"] + 4 * a.size].copy_(torch.from_numpy(a.view(np.uint8)))

    # -- readback -------------------------------------------------------------
    def read(self, off: int, nbytes: int) -> np.ndarray:
        self.synchronize()
        return self.blob[off:off + nbytes].cpu().numpy()

    def stage(self, name: str, rows: int, row0: int = 0) -> np.ndarray:
        """Rows of a stage buffer (h, h8, hs, q8, qs, o8, os, s8, ss, x, ...)."""
        L = self.layout
        H, I, QW, NH, KW = L.hidden, L.inter, L.q_width, L.heads, L.kv_width
        spec = {"x": ("kX", np.float32, H), "h": ("kH", np.float32, H),
                "h8": ("kH8", np.int8, H), "hs": ("kHS", np.float32, H // 256),
                "q8": ("kQ8", np.int8, QW), "qs": ("kQS", np.float32, NH),
                "o8": ("kO8", np.int8, QW), "os": ("kOS", np.float32, NH),
                "o": ("kO", np.float32, H), "s8": ("kS8", np.int8, I),
                "ss": ("kSS", np.float32, I // 256), "q": ("kQ", np.float32, QW),
                "k": ("kK", np.float32, KW), "v": ("kV", np.float32, KW),
                "logits": ("kLOGITS", np.float32, L.vocab)}[name]
        key, dt, width = spec
        es = np.dtype(dt).itemsize
        off = L[key] + row0 * width * es
        return self.read(off, rows * width * es).view(dt).reshape(rows, width)

    def ids(self) -> np.ndarray:
        L = self.layout
        return self.read(L["kIDS"], 4 * L.max_seq).view(np.int32)

    def argmax(self) -> tuple[np.float32, int]:
        L = self.layout
        f = self.read(L["kARGF"], 4).view(np.float32)[0]
        i = int(self.read(L["kARGI"], 4).view(np.int32)[0])
        return f, i

    def page_table_host(self) -> np.ndarray:
        t = getattr(self, "page_table", None)
        if t is None:
            n = self.layout.max_seq // 32
            t = np.arange(n - 1, -1, -1, dtype=np.uint16)
        return t

    def kv_cache(self, layer: int, n_tokens: int) -> dict[str, np.ndarray]:
        """Layer's K/V rows and scales in logical token order (through the
        page table), like ref_qwen3.Cache."""
        L = self.layout
        o = L.offsets
        KW, NKV, MS = L.kv_width, L.kv_heads, L.max_seq
        base = o["kKV_BASE"] + layer * o["kKV_STRIDE"]
        raw = self.read(base, o["kKV_STRIDE"])
        k = raw[:MS * KW].view(np.int8).reshape(MS // 32, 32, KW)
        ks = raw[o["kKV_SOFF"]:o["kKV_SOFF"] + 4 * MS * NKV].view(np.float32).reshape(MS // 32, 32, NKV)
        vo = o["kKV_VOFF"]
        v = raw[vo:vo + MS * KW].view(np.int8).reshape(MS // 32, 32, KW)
        vs = raw[vo + o["kKV_SOFF"]:vo + o["kKV_SOFF"] + 4 * MS * NKV].view(np.float32).reshape(
            MS // 32, 32, NKV)
        tab = self.page_table_host()
        t = np.arange(n_tokens)
        pages, slots = tab[t // 32], t % 32
        return {"kc": k[pages, slots], "ks": ks[pages, slots], "vc": v[pages, slots],
                "vs": vs[pages, slots]}
