"""The llm/runtime.py API on the MI355X datapath: LlamaDevice and run.c's Sampler.

    dev = LlamaDevice("stories15M_d16.w8a8", "tokenizer.bin")
    for tok, text in dev.generate("Once upon a time", steps=64, temperature=0.8, topp=0.9):
        print(text, end="", flush=True)
    dev.close()

Same methods, arguments, yields and exceptions as the reference's LlamaDevice
(llm/runtime.py:75-152): reset() empties the KV cache, forward(token) returns a float32 copy of
the logits and advances pos (ValueError when the sequence is full, RuntimeError when a step
fails), generate() feeds the prompt through the decode path and then samples. The FPGA-only
constructor arguments (bitfile, firmware, use_irq) are accepted and ignored; `device` names the
GPU ("cuda:0") instead of an injectable PYNQ Device.

Models: the reference's .w8a8 files (version 1; version 2, this package's extension, for
q_dim != dim, QK-norm and MoE), llama2.c fp32 checkpoints (quantised on load), a config name
(synthetic weights) or a QuantModel. Tokenizers: llama2.c tokenizer.bin (the default, next to
the model file) and HuggingFace tokenizer.json (t2r_amd.modelfile). Additions: prefill() runs
prompt rows through the int8 MFMA GEMM path (bit-identical to feeding them one by one), and
greedy_on_device() runs a whole greedy loop without host round trips.
"""
import os
import time

import numpy as np

from . import config as C
from . import modelfile as MF
from . import weights as W
from .model import ResidentModel

F = np.float32
BOS = 1


class XorShiftStar:
    """run.c's random numbers: a 64-bit xorshift state (shifts right 12, left 25, right 27) whose
    output is the high half of its product with 0x2545F4914F6CDD1D; a uniform float in [0, 1) is
    that output's top 24 bits over 2^24. Seed 0 is replaced by 1 (an all-zero state never moves)."""
    M64 = (1 << 64) - 1

    def __init__(self, seed):
        self.state = (seed & self.M64) or 1

    def u32(self):
        s = self.state
        s ^= s >> 12
        s = (s ^ (s << 25)) & self.M64
        s ^= s >> 27
        self.state = s
        return (s * 0x2545F4914F6CDD1D & self.M64) >> 32

    def uniform(self):
        return (self.u32() >> 8) * 2.0 ** -24         # exact: 24 bits scaled by a power of two


def _first_above(cdf, x, stop):
    """The first index i <= stop with cdf[i] > x (x compared as float32), else stop: run.c's
    "return the first index whose running sum exceeds the coin" with its clamp to the last."""
    hit = np.flatnonzero(cdf[:stop + 1] > F(x))
    return int(hit[0]) if hit.size else stop


class Sampler:
    """llama2.c run.c's sampler (llm/runtime.py:37-72): temperature 0 takes the argmax (first on
    ties). Otherwise the logits over the temperature go through a float32 softmax and one uniform
    draw picks the token: by the running sum of every probability (multinomial) when topp is not in
    (0, 1), else from the nucleus. The nucleus holds the tokens whose probability is at least
    (1 - topp) / (n - 1), by descending probability with the lower id first on ties; it ends at the
    first token whose running sum passes topp, and the draw is scaled by that sum. `state` is the
    generator's 64-bit state, which advances once per sampled (non-argmax) token."""

    def __init__(self, temperature=0.0, topp=0.9, seed=1):
        self.temperature, self.topp = temperature, topp
        self.rng = XorShiftStar(seed)

    @property
    def state(self):
        return self.rng.state

    def probabilities(self, logits):
        """softmax(logits / temperature) in float32: the maximum subtracted, then exp, then each
        divided by the (pairwise float32) sum."""
        x = np.asarray(logits, F) / F(self.temperature)
        e = np.exp(x - x.max())
        return e / e.sum(dtype=F)

    def __call__(self, logits):
        if self.temperature == 0:
            return int(np.argmax(logits))
        p = self.probabilities(logits)
        u = self.rng.uniform()
        if not 0 < self.topp < 1:
            return _first_above(np.cumsum(p, dtype=F), u, p.size - 1)
        ids = np.flatnonzero(p >= (1.0 - self.topp) / (p.size - 1))
        ids = ids[np.lexsort((ids, -p[ids]))]          # descending probability, then ascending id
        run = np.cumsum(p[ids], dtype=F)
        end = _first_above(run, F(self.topp), ids.size - 1)
        return int(ids[_first_above(run, u * float(run[end]), end)])


def _default_tokenizer(model_path):
    """tokenizer.bin next to a model file (the reference's default, llm/runtime.py:80-84), or an HF model
    directory's tokenizer.json."""
    if not isinstance(model_path, str):
        return None
    if os.path.isdir(model_path):
        return model_path if os.path.exists(os.path.join(model_path, "tokenizer.json")) else None
    if os.path.isfile(model_path):
        guess = os.path.join(os.path.dirname(os.path.abspath(model_path)), "tokenizer.bin")
        return guess if os.path.exists(guess) else None
    return None


def _resolve_model(model):
    if isinstance(model, W.QuantModel):
        return model
    if isinstance(model, C.ModelConfig):
        return W.QuantModel(model)
    if isinstance(model, str):
        if os.path.isdir(model) and os.path.exists(os.path.join(model, "config.json")):
            return MF.read_hf(model)                       # HF checkpoint (compiler/frontend/qhf.py:97-181)
        if os.path.isfile(model):
            if model.endswith(".bin"):                     # llama2.c fp32 checkpoint: quantised here
                cfg, w = MF.read_llama2c(model)
                return MF.quant_model_from_fp32(cfg, w)
            return MF.read_w8a8(model)                      # the device file (llm/runtime.py:80)
        return W.QuantModel(C.get(model))
    raise TypeError(f"model: a .w8a8 / llama2.c .bin path, an HF model directory, a ModelConfig, a config name or a QuantModel, "
                    f"not {type(model).__name__}")


class LlamaDevice:
    def __init__(self, model_path, tokenizer_path=None, bitfile=None, firmware=None, use_irq=True, device=None,
                 max_rows=None, bos_id=None):
        self.qm = _resolve_model(model_path)
        c = self.cfg = self.qm.cfg
        self.d = c.D
        self.tok = None
        if tokenizer_path is None:
            tokenizer_path = _default_tokenizer(model_path)
        if tokenizer_path is not None:
            self.tok = MF.open_tokenizer(tokenizer_path, c.vocab, bos_id=bos_id)
        self.m = ResidentModel(self.qm, device=device or "cuda:0", max_rows=max_rows)
        self.pos = 0
        self.stats = []                          # per token: (pos, device ns, wall seconds)

    def reset(self):
        """Start a new sequence: empty KV cache, pos 0."""
        self.m.reset()
        self.pos = 0

    def forward(self, token, perf=False):
        """Logits (float32 copy) of token at the current position; advances pos."""
        c = self.cfg
        if self.pos >= c.seq_len:
            raise ValueError(f"sequence full ({c.seq_len} positions)")
        torch = self.m.torch
        t0 = time.perf_counter()
        if perf:
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            ev0.record()
        try:
            lg = self.m.decode(token, self.pos)
            if perf:
                ev1.record()
            logits = lg.cpu().numpy().copy()
        except RuntimeError as e:
            raise RuntimeError(f"pos {self.pos}: step failed: {e}") from e
        self.m.check_status(f"pos {self.pos}: list")       # RuntimeError("pos N: list failed, status 0x..")
        wall = time.perf_counter() - t0
        dev_ns = int(ev0.elapsed_time(ev1) * 1e6) if perf else None
        self.stats.append((self.pos, dev_ns, wall))
        self.pos += 1
        return logits

    def prefill(self, tokens):
        """Feed prompt rows at pos.. in one pass (the MFMA GEMM path); returns the last row's logits
        (float32 copy). Bit-identical to calling forward() on each token."""
        c = self.cfg
        if self.pos + len(tokens) > c.seq_len:
            raise ValueError(f"sequence full ({c.seq_len} positions)")
        lg = self.m.prefill(tokens, start=self.pos)
        out = lg.cpu().numpy().copy()
        self.m.check_status(f"pos {self.pos}: list")
        self.pos += len(tokens)
        return out

    def generate(self, prompt, steps=256, temperature=0.0, topp=0.9, seed=1, stop_at_bos=True, forced=None):
        """Yield (token, text piece) per generated token, run.c style: the prompt tokens are fed first,
        then sampled tokens until `steps` positions (or BOS). prompt: text (encoded by the loaded
        tokenizer, BOS first) or token ids; the text piece is None without a tokenizer. forced:
        teacher forcing, yields (argmax, logits) per position."""
        self.reset()
        if forced is None and isinstance(prompt, str):
            if self.tok is None:
                raise ValueError("a text prompt needs a tokenizer (tokenizer_path); pass token ids instead")
            prompt = self.tok.encode(prompt)
        toks = list(forced) if forced is not None else list(prompt)
        sample = Sampler(temperature, topp, seed)
        token = toks[0]
        for pos in range(min(steps, self.cfg.seq_len)):
            logits = self.forward(token)
            if forced is not None:
                yield int(np.argmax(logits)), logits
                if pos + 1 >= len(forced):
                    return
                token = forced[pos + 1]
                continue
            nxt = toks[pos + 1] if pos + 1 < len(toks) else sample(logits)
            if nxt == BOS and stop_at_bos:
                return
            yield nxt, self._piece(token, nxt)
            token = nxt

    def _piece(self, token, nxt):
        """The text nxt adds after token (llm/runtime.py:146: decode of the pair minus decode of token)."""
        if self.tok is None:
            return None
        return self.tok.decode([token, nxt])[len(self.tok.decode([token])):]

    def greedy_on_device(self, prompt, steps, use_prefill=True):
        """Prompt (prefilled, or fed as decode steps), then greedy decode until `steps` positions, with
        the argmax and the position update on the device (no host round trip per token). Returns the
        tokens fed at every position plus the last one chosen (as ref_model.generate without BOS stop)."""
        torch = self.m.torch
        self.reset()
        P = len(prompt)
        steps = min(steps, self.cfg.seq_len)
        out = list(prompt[:steps])
        if use_prefill and P > 1:
            self.m.prefill(prompt[:min(P, steps)], start=0)
            self.m.tok.copy_(self.m.next)
            self.m.pos.fill_(min(P, steps))
            done = min(P, steps)
        else:
            done = 0
            for pos in range(min(P, steps)):
                self.m.decode(prompt[pos], pos)
            done = min(P, steps)
            self.m.tok.copy_(self.m.next)
            self.m.pos.fill_(done)
        gen = torch.empty(max(steps - done, 0) + 1, dtype=torch.int32, device=self.m.device)
        gen[0:1].copy_(self.m.tok)
        for i in range(steps - done):
            self.m.step(logits=False, advance=True)
            gen[i + 1:i + 2].copy_(self.m.tok)
        self.pos = steps
        g = gen.cpu().numpy().tolist()
        self.m.check_status(f"pos {done}..{steps - 1}: list")
        if done < P:
            return out
        return out + g[:steps - done + 1]

    def close(self):
        self.m.close()


class BatchLlamaDevice:
    """Batched decode (llm/runtime.py:155-245): `slots` sequences per step, each with its own KV
    cache and position; step() runs one token of every slot through t2r_decode_batch (the linear
    layers once over all rows on the int8 matrix cores, attention per row). A slot without a
    sequence runs a dummy token (BOS) at pos 0; its KV row 0 is rewritten when a sequence starts in
    it. Every row is bit-identical to the same token of that sequence run alone. slots defaults to
    the model's D, the reference's batch width."""
    DUMMY = BOS

    def __init__(self, model_path, tokenizer_path=None, bitfile=None, firmware=None, use_irq=True, device=None,
                 slots=None, bos_id=None):
        self.qm = _resolve_model(model_path)
        c = self.cfg = self.qm.cfg
        self.d = int(slots or c.D)
        self.tok = None
        if tokenizer_path is None:
            tokenizer_path = _default_tokenizer(model_path)
        if tokenizer_path is not None:
            self.tok = MF.open_tokenizer(tokenizer_path, c.vocab, bos_id=bos_id)
        self.m = ResidentModel(self.qm, device=device or "cuda:0", max_rows=self.d)
        self.kc, self.vc = self.m.batch_caches(self.d)
        self.stats = []                          # per step: (device ns or None, wall seconds)

    def clear_slot(self, b):
        """Empty slot b's KV cache."""
        self.kc[b].zero_()
        self.vc[b].zero_()

    def step(self, poses, tokens, perf=False):
        """One token for each of the slots; returns the (slots, vocab) logits (float32 copy)."""
        if len(poses) != self.d or len(tokens) != self.d:
            raise ValueError(f"one position and one token per slot ({self.d})")
        torch = self.m.torch
        t0 = time.perf_counter()
        if perf:
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            ev0.record()
        try:
            lg = self.m.decode_batch(tokens, poses, self.kc, self.vc)
            if perf:
                ev1.record()
            out = lg.cpu().numpy().copy()
        except RuntimeError as e:
            raise RuntimeError(f"step failed: {e}") from e
        self.m.check_status("step")                        # RuntimeError("step failed, status 0x..")
        self.stats.append((int(ev0.elapsed_time(ev1) * 1e6) if perf else None, time.perf_counter() - t0))
        return out

    def generate(self, prompts, steps, stagger=0, temperature=0.0, topp=0.9, seed=1, on_logits=None):
        """Generate for len(prompts) <= slots sequences at once; sequence b starts at step b * stagger
        and runs `steps` positions (prompt tokens fed first, then sampled; BOS does not stop it).
        prompts: texts (with a tokenizer) or token lists. on_logits(b, pos, logits) sees every
        position. Returns the token lists."""
        d = self.d
        n = len(prompts)
        if n > d:
            raise ValueError(f"at most {d} sequences")
        toks = []
        for p in prompts:
            if isinstance(p, str):
                if self.tok is None:
                    raise ValueError("text prompts need a tokenizer (tokenizer_path)")
                p = self.tok.encode(p)
            toks.append(list(p))
        steps = min(steps, self.cfg.seq_len)
        samplers = [Sampler(temperature, topp, seed + b) for b in range(n)]
        out = [[t[0]] for t in toks]
        start = [b * stagger for b in range(n)]
        for b in range(d):
            self.clear_slot(b)
        total = max(start) + steps if n else 0
        for s in range(total):
            poses, cur, live = [0] * d, [self.DUMMY] * d, [False] * d
            for b in range(n):
                p = s - start[b]
                if 0 <= p < steps:
                    poses[b], cur[b], live[b] = p, out[b][p], True
            logits = self.step(poses, cur)
            for b in range(n):
                if not live[b]:
                    continue
                p = poses[b]
                if on_logits:
                    on_logits(b, p, logits[b])
                if p + 1 < steps:
                    out[b].append(toks[b][p + 1] if p + 1 < len(toks[b]) else samplers[b](logits[b]))
        return out

    def close(self):
        self.m.close()

