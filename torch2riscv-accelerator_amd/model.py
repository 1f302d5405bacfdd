"""A W8A8 decoder resident on one MI355X, driven through the C-ABI (t2r_model_* in include/t2r.h).

PyTorch owns the device memory (weights, the int8 KV cache, the workspace, the per-step
(pos, token) block); the kernels are the HIP ones in libt2r.so. One decode step is one call to
t2r_decode_step, which reads the token and the position from device memory, so a HIP graph of
it replays unchanged step after step: the GPU form of the reference's static token list where
only the PARAM block and the (pos, token) arguments change (llm/compile_model.py:1-8, 56-62).
"""
import ctypes

import numpy as np

from . import abi

F = np.float32


class ResidentModel:
    def __init__(self, qm, device="cuda:0", max_rows=None, D=None, static_workspace=False):
        """qm: t2r_amd.weights.QuantModel (host arrays). max_rows: prefill rows per t2r_prefill call.
        static_workspace: the library's static workspace array instead of one allocated here
        (t2r_model_create_static; calls of such models on one device must not overlap)."""
        import torch
        self.torch = torch
        self.cfg = c = qm.cfg
        self.D = D or c.D
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError(f"{device}: the datapath runs on a GPU (HIP) device")
        if not torch.cuda.is_available():
            raise RuntimeError("no HIP device is visible: the W8A8 datapath has no CPU fallback")
        self.lib = abi.load()
        self.max_rows = max(1, int(max_rows or min(c.seq_len, 512)))
        dev = self.device
        keep = self._keep = {}

        def up(name, a):
            if a is None:
                return None
            t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
            keep[name] = t
            return t

        with torch.cuda.device(dev):
            up("emb_q", qm.emb_q); up("emb_s", qm.emb_s)
            # a tied classifier shares the embedding's int8 rows; its scales are its own when the logits'
            # scaling is folded into them
            if qm.cls_q is qm.emb_q:
                keep["cls_q"] = keep["emb_q"]
            else:
                up("cls_q", qm.cls_q)
            if qm.cls_s is qm.emb_s:
                keep["cls_s"] = keep["emb_s"]
            else:
                up("cls_s", qm.cls_s)
            for n in ("rms_att", "rms_ffn", "rms_final", "wqkv", "s_wqkv", "wo", "s_wo"):
                up(n, getattr(qm, n))
            if c.qk_norm:
                up("q_norm", qm.q_norm); up("k_norm", qm.k_norm)
            names = ("router", "s_router", "wg", "s_wg", "wu", "s_wu", "wd", "s_wd") if c.moe else \
                ("w1", "s_w1", "w3", "s_w3", "w2", "s_w2")
            for n in names:
                up(n, getattr(qm, n))
            up("rope_cos", qm.cos); up("rope_sin", qm.sin)
            kvch = getattr(qm, "kvch", None)
            self.kv_flags = np.ascontiguousarray(getattr(qm, "kv_flags", np.zeros(c.layers)), np.int32)
            if kvch is not None and self.kv_flags.any():
                up("kv_channel", kvch)
            self.kc = torch.zeros((c.layers, c.seq_len, c.kv_dim), dtype=torch.int8, device=dev)
            self.vc = torch.zeros_like(self.kc)
            self.kv_consts = np.ascontiguousarray(qm.kvc, F)
            desc = abi.ModelDesc()
            desc.abi_version = abi.T2R_ABI_VERSION
            desc.dim, desc.hidden, desc.layers = c.dim, c.hidden, c.layers
            desc.heads, desc.kv_heads, desc.head_dim = c.heads, c.kv_heads, c.head_dim
            desc.vocab, desc.seq_len = c.vocab, c.seq_len
            desc.n_experts, desc.top_k = c.n_experts, c.top_k
            desc.qk_norm, desc.D, desc.eps = int(c.qk_norm), self.D, float(F(c.eps))
            for n, t in keep.items():
                setattr(desc, n, t.data_ptr())
            desc.kv_consts = self.kv_consts.ctypes.data
            desc.attn_qsum = int(c.attn_norm == "qsum")
            desc.ffn_act = int(c.act == "gelu_tanh")
            desc.kv_channel_flags = self.kv_flags.ctypes.data
            desc.k_cache, desc.v_cache = self.kc.data_ptr(), self.vc.data_ptr()
            desc.max_rows = self.max_rows
            nbytes = self.lib.t2r_model_workspace_bytes(ctypes.byref(desc), self.max_rows)
            if nbytes <= 0:
                raise ValueError("t2r_model_workspace_bytes rejected the model description")
            self.desc = desc
            handle = ctypes.c_void_p()
            if static_workspace:
                self.workspace = None
                desc.workspace, desc.workspace_bytes = None, 0
                abi.check("t2r_model_create_static",
                          self.lib.t2r_model_create_static(ctypes.byref(desc), ctypes.byref(handle)))
            else:
                self.workspace = torch.empty(int(nbytes), dtype=torch.uint8, device=dev)
                desc.workspace, desc.workspace_bytes = self.workspace.data_ptr(), int(nbytes)
                abi.check("t2r_model_create", self.lib.t2r_model_create(ctypes.byref(desc), ctypes.byref(handle)))
            self.handle = handle
            self.tok = torch.zeros(1, dtype=torch.int32, device=dev)
            self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
            self.next = torch.zeros(1, dtype=torch.int32, device=dev)
            self.logits = torch.empty(c.vocab, dtype=torch.float32, device=dev)
            self.rows_tok = torch.zeros(self.max_rows, dtype=torch.int32, device=dev)
            self.rows_pos = torch.zeros(self.max_rows, dtype=torch.int32, device=dev)

    # ------------------------------------------------------------ state
    def reset(self):
        """Empty KV cache (rows beyond pos must be zero, as the reference's runtime keeps them)."""
        self.kc.zero_()
        self.vc.zero_()

    def close(self):
        if getattr(self, "handle", None):
            self.lib.t2r_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ------------------------------------------------------------ steps
    def step(self, logits=True, advance=False, stream=None):
        """One decode step on the device-resident (self.tok, self.pos); the greedy token goes to self.next
        (or to self.tok and pos += 1 with advance=True, for a device-side greedy loop)."""
        nxt = self.tok if advance else self.next
        abi.check("t2r_decode_step", self.lib.t2r_decode_step(
            self.handle, abi.ptr(self.tok), abi.ptr(self.pos), abi.ptr(self.logits) if logits else None,
            abi.ptr(nxt), abi.T2R_ADVANCE_POS if advance else 0, abi.stream_ptr(stream)))

    def decode(self, token, pos):
        """Logits (device tensor, valid until the next call) of `token` at `pos`."""
        if not 0 <= pos < self.cfg.seq_len:
            raise ValueError(f"position {pos} outside [0, {self.cfg.seq_len})")
        self._check_tokens([token])
        self.tok.fill_(int(token))
        self.pos.fill_(int(pos))
        self.step()
        return self.logits

    def _check_tokens(self, tokens):
        bad = [int(t) for t in tokens if not 0 <= int(t) < self.cfg.vocab]
        if bad:
            raise ValueError(f"token {bad[0]} outside [0, {self.cfg.vocab})")

    def status(self, clear=True):
        """The device status word (bit 0: a token outside the vocabulary was embedded; bit 1: a bounded
        wait between the workgroups of a head's split decode attention ran out; bit 2: a row's position
        was outside the cache); waits for the device."""
        out = np.zeros(1, np.int32)
        abi.check("t2r_model_status", self.lib.t2r_model_status(self.handle, out.ctypes.data, int(clear)))
        return int(out[0])

    def check_status(self, where):
        """The reference's check after every list (llm/runtime.py:118-119, 202-203): a non-zero status
        word raises RuntimeError(f"{where} failed, status {s:#x}") and is cleared, so the next call starts
        clean. Waits for the device (the caller is about to read results anyway)."""
        s = self.status(clear=False)
        if s:
            self.status(clear=True)
            raise RuntimeError(f"{where} failed, status {s:#x}")

    def prefill(self, tokens, start=0, logits=True):
        """Rows tokens at positions start.. as one call per max_rows chunk; logits of the last row."""
        torch = self.torch
        toks = [int(t) for t in tokens]
        if start < 0 or start + len(toks) > self.cfg.seq_len:
            raise ValueError(f"positions {start}..{start + len(toks) - 1} outside [0, {self.cfg.seq_len})")
        if not toks:
            raise ValueError("empty prompt")
        self._check_tokens(toks)
        i = 0
        while i < len(toks):
            chunk = toks[i:i + self.max_rows]
            M = len(chunk)
            self.rows_tok[:M].copy_(torch.tensor(chunk, dtype=torch.int32))
            last = i + M >= len(toks)
            abi.check("t2r_prefill_at", self.lib.t2r_prefill_at(
                self.handle, abi.ptr(self.rows_tok), start + i, M,
                abi.ptr(self.logits) if (last and logits) else None, abi.ptr(self.next) if last else None,
                abi.stream_ptr()))
            i += M
        return self.logits

    def batch_caches(self, B):
        """Zeroed KV caches for B sequences of decode_batch: two int8 tensors (B, layers, seq_len, kv_dim)."""
        c = self.cfg
        kc = self.torch.zeros((B, c.layers, c.seq_len, c.kv_dim), dtype=self.torch.int8, device=self.device)
        return kc, self.torch.zeros_like(kc)

    def decode_batch(self, tokens, positions, kc, vc, logits=None, next_tokens=None):
        """One decode token of each of B sequences (t2r_decode_batch): row b is tokens[b] at
        positions[b] with the caches kc[b] / vc[b] (batch_caches). Returns the logits [B, vocab]
        (a device tensor: `logits` when given); next_tokens, when given, receives each row's argmax."""
        torch = self.torch
        B = len(tokens)
        if not 1 <= B <= self.max_rows:
            raise ValueError(f"{B} sequences: between 1 and max_rows = {self.max_rows}")
        if len(positions) != B or kc.shape[0] < B or vc.shape != kc.shape:
            raise ValueError("one position and one cache per sequence")
        c = self.cfg
        if kc.shape[1:] != (c.layers, c.seq_len, c.kv_dim) or kc.dtype != torch.int8 or not kc.is_contiguous():
            raise ValueError("caches: contiguous int8 (B, layers, seq_len, kv_dim), as batch_caches makes them")
        pos = [int(p) for p in positions]
        if min(pos) < 0 or max(pos) >= c.seq_len:
            raise ValueError(f"positions outside [0, {c.seq_len})")
        self._check_tokens(tokens)
        self.rows_tok[:B].copy_(torch.tensor([int(t) for t in tokens], dtype=torch.int32))
        self.rows_pos[:B].copy_(torch.tensor(pos, dtype=torch.int32))
        out = logits if logits is not None else torch.empty((B, c.vocab), dtype=torch.float32, device=self.device)
        abi.check("t2r_decode_batch", self.lib.t2r_decode_batch(
            self.handle, abi.ptr(self.rows_tok), abi.ptr(self.rows_pos), B, abi.ptr(kc), abi.ptr(vc),
            kc[0].numel(), abi.ptr(out), abi.ptr(next_tokens), abi.stream_ptr()))
        return out

    def prefill_chunks(self, tokens, M=16):
        """The reference's chunk schedule (compiler/frontend/export.py:69-72): chunks of M rows at
        0, M, 2M, ... and a last one at P - M (it recomputes rows the one before wrote, with the same
        values); a prompt shorter than M runs as one chunk."""
        P = len(tokens)
        starts = [0] if P <= M else list(range(0, P - M, M)) + [P - M]
        out = None
        for s in starts:
            out = self.prefill(tokens[s:s + M], start=s)
        return out

    # ------------------------------------------------------------ timing
    def profile(self, kinds=("qkv", "attn", "wo", "ffn_up", "ffn_down", "cls", "route", "other"), max_launches=65536):
        """Record HIP events around every launch of these kernel classes from now on (t2r_model_profile);
        kinds=() stops recording and frees the events."""
        mask = 0
        for k in kinds:
            mask |= 1 << abi.PROF_KINDS.index(k)
        abi.check("t2r_model_profile", self.lib.t2r_model_profile(self.handle, mask, max_launches if mask else 0))
        self._prof_max = max_launches if mask else 0

    def profile_read(self):
        """{kind: [ms of each recorded launch]} since the last read (waits for the recorded events)."""
        n = getattr(self, "_prof_max", 0)
        kinds = np.zeros(max(n, 1), np.int32)
        ms = np.zeros(max(n, 1), np.float32)
        got = self.lib.t2r_model_profile_read(self.handle, kinds.ctypes.data, ms.ctypes.data, n)
        if got < 0:
            abi.check("t2r_model_profile_read", got)
        out = {}
        for k, t in zip(kinds[:got], ms[:got]):
            out.setdefault(abi.PROF_KINDS[k], []).append(float(t))
        return out

    # ------------------------------------------------------------ HIP graphs
    def capture_decode(self, steps):
        """A HIP graph of `steps` greedy decode steps on the device-resident (tok, pos): each replay
        runs them with the argmax and pos += 1 on the device and no host work. Replaying it again
        continues from wherever (tok, pos) stand. Kernel timing (profile()) is switched off for the
        capture: events recorded during stream capture cannot be timed afterwards."""
        torch = self.torch
        if getattr(self, "_prof_max", 0):
            self.profile(kinds=())
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        tok, pos = self.tok.clone(), self.pos.clone()
        with torch.cuda.stream(side):
            self.step(logits=False, advance=True)          # one eager step on the capture stream first
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        with torch.cuda.graph(g, stream=side):
            for _ in range(steps):
                self.step(logits=False, advance=True)
        self.tok.copy_(tok)
        self.pos.copy_(pos)
        torch.cuda.synchronize(self.device)
        return g

    def capture_prefill(self, tokens, start=0):
        """A HIP graph of one prefill call (t2r_prefill_at) of `tokens` (at most max_rows) at positions
        start..: the token ids are copied to the device first, so each replay runs the prompt's layers
        with no host work (the prefill's ~8 launches a layer replayed at once); the last row's logits go
        to self.logits and its greedy token to self.next. The KV rows are rewritten by every replay.
        Kernel timing is switched off, as for capture_decode."""
        torch = self.torch
        toks = [int(t) for t in tokens]
        M = len(toks)
        if not 1 <= M <= self.max_rows or start < 0 or start + M > self.cfg.seq_len:
            raise ValueError(f"{M} rows at {start}: 1..max_rows = {self.max_rows} rows inside the cache")
        self._check_tokens(toks)
        if getattr(self, "_prof_max", 0):
            self.profile(kinds=())
        self.rows_tok[:M].copy_(torch.tensor(toks, dtype=torch.int32))
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))

        def call(st):
            abi.check("t2r_prefill_at", self.lib.t2r_prefill_at(
                self.handle, abi.ptr(self.rows_tok), int(start), M, abi.ptr(self.logits), abi.ptr(self.next),
                abi.stream_ptr(st)))
        with torch.cuda.stream(side):
            call(side)                                  # one eager call on the capture stream first
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        with torch.cuda.graph(g, stream=side):
            call(side)
        torch.cuda.synchronize(self.device)
        return g
