"""Host side of the HIP decode engine.

``HipEngine`` wraps one engine handle of libpulsar_hip.so (a batch of sequences with its KV
cache). ``PulsarInferenceEngine`` mirrors the reference's generation interface
(src/infer.py:181-782: ``generate``, ``stream_generate``, ``self_speculative_stream_generate``)
and adds a batched id-level entry, ``generate_ids``.

The whole decode loop runs on the GPU: each step is one pulse of every active row, the
sampling and the accept/resample controller included, replayed from a captured HIP graph;
the host only polls a done flag every few steps.
"""

from __future__ import annotations

import ctypes
from typing import Iterable, Iterator, Optional, Sequence

import numpy as np
import torch

from pulsar_cuda import _lib

from .model import DeviceModel

# Seq-state fields (int32 words of the controller's per-sequence record).
ST_DONE, ST_PRODUCED, ST_TESTS, ST_ACCEPTED = 0, 1, 11, 12


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


class HipEngine:
    """A batch of sequences decoded by the HIP engine."""

    def __init__(self, model: DeviceModel, *, batch: int, max_prompt: int, max_new: int,
                 speculative: bool = True, temperature: float = 0.7, top_p: float = 0.9,
                 repetition_penalty: float = 1.15, stop_ids: Iterable[int] = (0,),
                 seed: int = 0, all_logits: bool = False, max_ctx: Optional[int] = None,
                 draft_len: int = 0, early_exit_threshold: Optional[float] = None,
                 kv_pages: Optional[int] = None):
        """draft_len = 0 runs the reference's exact self-speculation; 1..7 the draft-block
        mode (up to draft_len pulse-0 drafts per round, one all-pulse verify of the block).
        early_exit_threshold (exact schedule only): the reference's adaptive early exit
        (src/infer.py:536-547); None switches it off. kv_pages: pages of 64 positions in the
        global layers' KV pool shared by the batch (None: enough for every sequence to
        reach max_ctx); sequences take pages as they reach them, and run() raises when a
        sequence found the pool spent."""
        self.lib = _lib.load()
        self.model = model
        self.batch = batch
        self.max_new = max_new
        self.draft_len = int(draft_len)
        # rows of one sequence in a step: 2 in the exact schedule; the block (+ the next
        # round's first row when it fits the 8 rows of an attention unit) in the draft-block
        # mode (engine_slots in csrc/sample.h)
        g = self.draft_len
        self.slots = 2 if g <= 0 else (g + 2 if g + 2 <= 8 else g + 1)
        self.V = model.cfg.vocab_size
        stops = sorted({int(s) for s in stop_ids})
        if len(stops) > 8:
            raise ValueError(f"at most 8 stop ids are supported, got {len(stops)}")
        c = _lib.PulsarEngineConfig()
        c.max_batch, c.max_prompt, c.max_new = batch, max_prompt, max_new
        c.max_ctx = max_ctx or (max_prompt + max_new + 2 + self.draft_len)
        c.draft_len = self.draft_len
        c.speculative, c.all_logits = int(bool(speculative)), int(bool(all_logits))
        c.temperature, c.top_p, c.repetition_penalty = temperature, top_p, repetition_penalty
        c.n_stop = len(stops)
        for i, s in enumerate(stops):
            c.stop_ids[i] = s
        c.seed = seed & 0xFFFFFFFFFFFFFFFF
        c.early_exit = int(early_exit_threshold is not None)
        c.early_exit_threshold = float(early_exit_threshold) if early_exit_threshold is not None else 0.0
        c.kv_pages = int(kv_pages or 0)
        self.early_exit_threshold = early_exit_threshold
        model.ensure_rope(c.max_ctx)
        self.cfg = c
        h = ctypes.c_void_p()
        _lib.check(self.lib.pulsar_engine_create(model.desc_ref(), ctypes.byref(c), ctypes.byref(h)))
        self.handle = h
        self.steps = 0

    def close(self) -> None:
        if self.handle:
            self.lib.pulsar_engine_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- running ---------------------------------------------------------------
    def prefill(self, ids) -> None:
        a = np.ascontiguousarray(np.asarray(ids, dtype=np.int32))
        if a.ndim != 2 or a.shape[0] != self.batch:
            raise ValueError(f"prompt ids must be [batch={self.batch}, T]")
        _lib.check(self.lib.pulsar_engine_prefill(self.handle, a.ctypes.data, a.shape[0],
                                                  a.shape[1], _stream()))
        self.steps = 0

    def fill_kv(self, ctx: int, seed: int = 0) -> None:
        """Synthetic cache: every cached key/value element ~ N(0, 1); positions [0, ctx)
        then count as context for verify()."""
        _lib.check(self.lib.pulsar_engine_fill_kv(self.handle, int(ctx), seed & 0xFFFFFFFFFFFFFFFF,
                                                  _stream()))

    def verify(self, tokens=None, graph: bool = False) -> None:
        """Block verify of tokens [batch, n] at the positions after the cached context,
        through every pulse; the last pulse's logits are then readable with logits(batch*n)
        (row b*n + i). tokens=None re-runs the last block (no host synchronisation)."""
        if tokens is None:
            _lib.check(self.lib.pulsar_engine_verify(self.handle, None, 0, int(graph), _stream()))
            return
        a = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32))
        if a.ndim != 2 or a.shape[0] != self.batch:
            raise ValueError(f"verify tokens must be [batch={self.batch}, n]")
        _lib.check(self.lib.pulsar_engine_verify(self.handle, a.ctypes.data, a.shape[1],
                                                 int(graph), _stream()))

    def rewind(self, seed: int) -> None:
        """Restart decoding from the prefilled cache with a new sampling seed."""
        _lib.check(self.lib.pulsar_engine_rewind(self.handle, seed & 0xFFFFFFFFFFFFFFFF, _stream()))
        self.steps = 0

    def profile(self, enable: bool) -> None:
        """Per-kernel-class HIP-event timing; steps run eagerly while enabled, with a short
        fixed sleep kernel ahead of each timed kernel group so that its events bracket the
        kernels rather than host launch latency."""
        _lib.check(self.lib.pulsar_engine_profile(self.handle, int(bool(enable))))

    def profile_read(self) -> dict:
        ms = (ctypes.c_double * _lib.PROF_CLASSES)()
        n = (ctypes.c_int64 * _lib.PROF_CLASSES)()
        _lib.check(self.lib.pulsar_engine_profile_read(self.handle, ms, n))
        return {name: (ms[i], n[i]) for i, name in enumerate(_lib.PROF_NAMES)}

    def step(self, n: int = 1, graph: bool = False) -> None:
        _lib.check(self.lib.pulsar_engine_step(self.handle, n, int(graph), _stream()))
        self.steps += n

    def run(self, max_steps: Optional[int] = None, check_every: int = 16) -> int:
        """Step until every sequence finished; returns the number of steps run."""
        if max_steps is None:
            max_steps = 4 * (self.max_new + 2) * (self.model.n_pulses + self.draft_len)
        ran = ctypes.c_int32(0)
        _lib.check(self.lib.pulsar_engine_generate(self.handle, max_steps, check_every, _stream(),
                                                   ctypes.byref(ran)))
        self.steps += ran.value
        pages = self.kv_pages()
        if pages["spent"]:
            raise RuntimeError(f"KV page pool spent ({pages['pool']} pages): sequences that "
                               f"needed another page stopped early")
        return ran.value

    # -- reading ---------------------------------------------------------------
    def _read(self, what: int, arr: np.ndarray) -> np.ndarray:
        _lib.check(self.lib.pulsar_engine_read(self.handle, what, arr.ctypes.data, arr.nbytes,
                                               _stream()))
        return arr

    def state(self) -> np.ndarray:
        return self._read(_lib.BUF_SEQSTATE, np.zeros((self.batch, _lib.SEQSTATE_INTS), np.int32))

    def tokens(self) -> list[list[int]]:
        st = self.state()
        toks = self._read(_lib.BUF_TOKENS, np.zeros((self.batch, max(1, self.max_new)), np.int32))
        return [toks[b, : st[b, ST_PRODUCED]].tolist() for b in range(self.batch)]

    def ctl(self) -> np.ndarray:
        """Control block of the next step: n_rows, n_lrows, pulse_start[4], pulse_count[4],
        active sequences, step counter."""
        return self._read(_lib.BUF_CTL, np.zeros(_lib.CTL_INTS, np.int32))

    def last_ctl(self) -> np.ndarray:
        """Control block of the last executed step."""
        return self._read(_lib.BUF_LAST_CTL, np.zeros(_lib.CTL_INTS, np.int32))

    def logits(self, n: int) -> np.ndarray:
        return self._read(_lib.BUF_LOGITS, np.zeros((n, self.V), np.float32))

    def rows(self, last: bool = True) -> np.ndarray:
        """Rows (seq, slot, pulse, pos, token, lrow, extra, 0) of the last executed step, or of
        the next step when last=False."""
        ctl = self._read(_lib.BUF_LAST_CTL if last else _lib.BUF_CTL,
                         np.zeros(_lib.CTL_INTS, np.int32))
        buf = np.zeros((self.slots * self.batch, _lib.ROW_INTS), np.int32)
        self._read(_lib.BUF_LAST_ROWS if last else _lib.BUF_ROWS, buf)
        return buf[: int(ctl[0])]

    def expert_counts(self) -> np.ndarray:
        """Rows routed to each expert in every layer during the last step, [layers, E]."""
        c = self.model.cfg
        return self._read(_lib.BUF_EXPERT_COUNTS, np.zeros((c.n_core, c.n_routed_experts), np.int32))

    def acceptance(self) -> tuple[int, int]:
        st = self.state()
        return int(st[:, ST_TESTS].sum()), int(st[:, ST_ACCEPTED].sum())

    def token_kinds(self) -> list[list[int]]:
        """Per emitted token: 1 when it was an accepted draft, 0 when drawn (the first token,
        a plain draw, or the fresh draw after a rejected draft)."""
        st = self.state()
        k = self._read(_lib.BUF_TOKEN_KINDS, np.zeros((self.batch, max(1, self.max_new)), np.int32))
        return [k[b, : st[b, ST_PRODUCED]].tolist() for b in range(self.batch)]

    def kv_layout(self) -> dict:
        """Cache layout: ring positions of a sliding-window layer, page-table entries per
        sequence of a global layer, positions per page, kv heads."""
        v = self._read(_lib.BUF_KV_LAYOUT, np.zeros(4, np.int32))
        return {"lcap": int(v[0]), "max_pages": int(v[1]), "page": int(v[2]), "hkv": int(v[3])}

    def kv_pages(self) -> dict:
        """Global-layer KV pages: pool size, pages handed out, whether a request found the
        pool spent (since the last prefill, fill_kv or rewind)."""
        v = self._read(_lib.BUF_KV_PAGES, np.zeros(3, np.int32))
        return {"pool": int(v[0]), "used": int(v[1]), "spent": bool(v[2])}

    def exit_counts(self) -> np.ndarray:
        """Early exit: tokens of each sequence that left after pulse k, [batch, n_pulses],
        since the last prefill or rewind."""
        c = self._read(_lib.BUF_EXIT_COUNTS, np.zeros((self.batch, 4), np.int32))
        return c[:, : self.model.n_pulses]

    def topk_idx(self) -> np.ndarray:
        """Router top-k expert ids of every row of the last executed step in every layer,
        [layers, rows, top_k] in the router's ranking order (rows as in rows())."""
        c = self.model.cfg
        buf = np.zeros((c.n_core, self.slots * self.batch, c.top_k), np.int32)
        self._read(_lib.BUF_TOPK_IDX, buf)
        n = int(self.last_ctl()[0])
        return buf[:, :n]


def sample_rows(logits: torch.Tensor, seen: Sequence[Iterable[int]], row_seq: Sequence[int],
                row_extra: Sequence[int], ctr: Sequence[int], seed: int, temperature: float,
                top_p: float, repetition_penalty: float, greedy: bool = False,
                dtype: torch.dtype = torch.bfloat16) -> tuple[np.ndarray, np.ndarray]:
    """The engine's sampling kernel on given fp32 logits rows (device tensor [n, V]).

    ``seen[s]`` are the token ids sequence s has seen, ``row_seq[i]`` the sequence of row i,
    ``row_extra[i]`` one more token counted as seen for row i (-1: none), ``ctr[s]`` the
    sequence's draw counter. Returns (penalised argmax [n], two draws per row [n, 2]),
    following the reference's _sample (src/infer.py:658-685) with the engine's generator."""
    lib = _lib.load()
    n, V = logits.shape
    dev = logits.device
    bits = np.zeros((len(seen), V // 32), dtype=np.uint32)
    for s_, ids in enumerate(seen):
        for t in set(int(x) for x in ids):
            bits[s_, t >> 5] |= np.uint32(1 << (t & 31))
    seen_d = torch.from_numpy(bits.view(np.int32)).to(dev)
    rs = torch.as_tensor(list(row_seq), dtype=torch.int32, device=dev)
    rx = torch.as_tensor(list(row_extra), dtype=torch.int32, device=dev)
    cd = torch.as_tensor(np.asarray(ctr, dtype=np.uint32).view(np.int32), device=dev)
    ws = torch.empty(int(lib.pulsar_sample_workspace_bytes(len(seen))), dtype=torch.uint8,
                     device=dev)
    am = torch.empty(n, dtype=torch.int32, device=dev)
    dr = torch.empty(n, 2, dtype=torch.int32, device=dev)
    lg = logits.contiguous().float()
    _lib.check(lib.pulsar_sample_rows(
        lg.data_ptr(), n, V, _lib.PULSAR_BF16 if dtype == torch.bfloat16 else _lib.PULSAR_F32,
        seen_d.data_ptr(), rs.data_ptr(), rx.data_ptr(), cd.data_ptr(), len(seen),
        seed & 0xFFFFFFFFFFFFFFFF, temperature, top_p, repetition_penalty, int(bool(greedy)),
        am.data_ptr(), dr.data_ptr(), ws.data_ptr(), _stream()))
    torch.cuda.synchronize(dev)
    return am.cpu().numpy(), dr.cpu().numpy()


def early_exit_stats(counts: Sequence[int]) -> dict:
    """Distribution of exit pulses (src/infer.py:215-232): per-pulse counts and shares, the
    effective depth with pulses weighed as 8, 16 and 24 layers, and 24 / depth."""
    c = [int(x) for x in counts]
    total = sum(c)
    if total == 0:
        return {}
    eff = (8 * c[0] + 16 * c[1] + 24 * c[2]) / total
    return {"total_tokens": total, "pulse_counts": c,
            "pulse_pcts": [c[0] / total * 100.0, c[1] / total * 100.0, c[2] / total * 100.0],
            "effective_layers": eff, "compute_speedup": 24.0 / eff}


def format_early_exit_stats(threshold: float, stats: dict) -> str:
    """The block generate() prints after the text when early exit is on (src/infer.py:775-780)."""
    p = stats["pulse_pcts"]
    return (f"\n[Adaptive Early-Exit Stats | Threshold: {threshold:.2f}]\n"
            f"  Tokens: {stats['total_tokens']} | P1 (8L): {p[0]:.1f}% | P2 (16L): {p[1]:.1f}% "
            f"| P3 (24L): {p[2]:.1f}%\n"
            f"  Effective Depth: {stats['effective_layers']:.1f} layers | "
            f"Speedup: {stats['compute_speedup']:.2f}x\n")


def stop_ids_for(cfg, tokenizer=None) -> set[int]:
    """{eos} plus the tokenizer ids of the reference's stop strings (src/infer.py:649-656)."""
    ids = {cfg.eos_token_id}
    if tokenizer is not None:
        for s in ("<|im_end|>", "<|endoftext|>", "</s>"):
            try:
                sid = tokenizer.convert_tokens_to_ids(s)
            except (KeyError, ValueError, TypeError):  # tokenizer without this token
                continue
            if sid is not None and sid != getattr(tokenizer, "unk_token_id", None):
                ids.add(int(sid))
    return ids


class PulsarInferenceEngine:
    """Generation interface of the reference engine on the HIP decode path."""

    def __init__(self, model: DeviceModel, device="cuda", dtype=None):
        self.model = model
        self.cfg = model.cfg
        self.device = torch.device(device)
        self.dtype = model.dtype
        self.stop_token_ids = {self.cfg.eos_token_id}
        self.last_engine: Optional[HipEngine] = None
        # adaptive early exit (src/infer.py:198-200): off until a threshold is set; the
        # counts add up over generations until the threshold is set again
        self.early_exit_threshold: Optional[float] = None
        self.early_exit_counts = [0] * model.n_pulses
        # engines (KV cache, buffers, captured graphs) kept for reuse, keyed by batch shape
        # and generation settings
        self._engines: dict = {}
        self.max_cached_engines = 4

    def set_early_exit_threshold(self, threshold: Optional[float]) -> None:
        """Confidence threshold of the adaptive early exit; clears the counts
        (src/infer.py:210-213)."""
        self.early_exit_threshold = threshold
        self.early_exit_counts = [0] * self.model.n_pulses

    def get_early_exit_stats(self) -> dict:
        """src/infer.py:215-232."""
        return early_exit_stats(self.early_exit_counts)

    def _engine(self, batch: int, prompt_len: int, max_new: int, speculative: bool,
                temperature: float, top_p: float, repetition_penalty: float, stops, seed: int,
                draft_len: int) -> HipEngine:
        key = (batch, prompt_len, max_new, bool(speculative), float(temperature), float(top_p),
               float(repetition_penalty), tuple(stops), int(draft_len),
               self.early_exit_threshold)
        eng = self._engines.get(key)
        if eng is None or eng.handle is None:
            while len(self._engines) >= self.max_cached_engines:
                self._engines.pop(next(iter(self._engines))).close()
            eng = HipEngine(self.model, batch=batch, max_prompt=prompt_len, max_new=max_new,
                            speculative=speculative, temperature=temperature, top_p=top_p,
                            repetition_penalty=repetition_penalty, stop_ids=stops, seed=seed,
                            draft_len=draft_len, early_exit_threshold=self.early_exit_threshold)
            self._engines[key] = eng
        return eng

    def _decode(self, eng: HipEngine, ids: np.ndarray, seed: int) -> None:
        """Prefill (first token drawn with the engine's creation seed) and, for another seed,
        redraw the first token from the kept prefill logits."""
        eng.prefill(ids)
        if (seed & 0xFFFFFFFFFFFFFFFF) != eng.cfg.seed:
            eng.rewind(seed)

    def _count_exits(self, eng: HipEngine) -> None:
        if self.early_exit_threshold is not None:
            c = eng.exit_counts().sum(axis=0)
            self.early_exit_counts = [a + int(b) for a, b in zip(self.early_exit_counts, c)]

    def generate_ids(self, prompt_ids: Sequence[Sequence[int]], max_new_tokens: int = 512,
                     temperature: float = 0.7, top_p: float = 0.9,
                     repetition_penalty: float = 1.15, speculative: bool = True,
                     stop_ids: Optional[Iterable[int]] = None, seed: int = 0,
                     draft_len: int = 0) -> list[list[int]]:
        """Batched id-level generation. Prompts of different lengths run as one batch per
        length (results in prompt order). draft_len > 0 selects the draft-block mode (no
        reference counterpart; see HipEngine)."""
        if len(prompt_ids) and np.ndim(prompt_ids[0]) == 0:
            prompt_ids = [prompt_ids]
        prompts = [np.asarray(p, dtype=np.int32).reshape(-1) for p in prompt_ids]
        stops = sorted(stop_ids if stop_ids is not None else self.stop_token_ids)
        groups: dict[int, list[int]] = {}
        for i, p in enumerate(prompts):
            if p.size == 0:
                raise ValueError("empty prompt")
            groups.setdefault(p.size, []).append(i)
        out: list = [None] * len(prompts)
        for T, members in groups.items():
            ids = np.stack([prompts[i] for i in members])
            eng = self._engine(len(members), T, max_new_tokens, speculative, temperature, top_p,
                               repetition_penalty, stops, seed, draft_len)
            self.last_engine = eng
            self._decode(eng, ids, seed)
            eng.run()
            self._count_exits(eng)
            for i, toks in zip(members, eng.tokens()):
                out[i] = toks
        return out

    def _stream(self, tokenizer, prompt: str, max_new_tokens, temperature, top_p,
                repetition_penalty, speculative) -> Iterator[str]:
        ids = tokenizer.encode(prompt, return_tensors="pt")
        ids = np.asarray(ids.reshape(1, -1).cpu().numpy(), dtype=np.int32)
        stops = stop_ids_for(self.cfg, tokenizer)
        eng = self._engine(1, ids.shape[1], max_new_tokens, speculative, temperature, top_p,
                           repetition_penalty, sorted(stops), 0, 0)
        self.last_engine = eng
        self._decode(eng, ids, 0)
        sent = 0
        limit = 4 * (max_new_tokens + 2) * self.model.n_pulses
        while True:
            toks = eng.tokens()[0]
            for t in toks[sent:]:
                yield tokenizer.decode([t], skip_special_tokens=False)
            sent = len(toks)
            if eng.state()[0, ST_DONE] or eng.steps >= limit:
                break
            eng.step(8, graph=True)
        self._count_exits(eng)

    def stream_generate(self, tokenizer, prompt: str, max_new_tokens: int = 512,
                        temperature: float = 0.7, top_p: float = 0.9,
                        repetition_penalty: float = 1.15) -> Iterator[str]:
        """Plain decode (src/infer.py:551-621)."""
        return self._stream(tokenizer, prompt, max_new_tokens, temperature, top_p,
                            repetition_penalty, speculative=False)

    def self_speculative_stream_generate(self, tokenizer, prompt: str, max_new_tokens: int = 512,
                                         temperature: float = 0.7, top_p: float = 0.9,
                                         repetition_penalty: float = 1.15) -> Iterator[str]:
        """Pulse-0 draft, last-pulse verify (src/infer.py:623-731)."""
        return self._stream(tokenizer, prompt, max_new_tokens, temperature, top_p,
                            repetition_penalty, speculative=True)

    def generate(self, tokenizer, prompt: str, max_new_tokens: int = 512,
                 temperature: float = 0.7, top_p: float = 0.9, repetition_penalty: float = 1.15,
                 stream: bool = False, speculative: bool = False) -> str:
        """Prompt plus completion, optionally streamed to stdout (src/infer.py:733-782)."""
        import sys

        gen = (self.self_speculative_stream_generate if speculative else self.stream_generate)(
            tokenizer, prompt, max_new_tokens=max_new_tokens, temperature=temperature,
            top_p=top_p, repetition_penalty=repetition_penalty)
        pieces = []
        for piece in gen:
            if stream:
                sys.stdout.write(piece)
                sys.stdout.flush()
            pieces.append(piece)
        if stream:
            sys.stdout.write("\n")
            sys.stdout.flush()
        if self.early_exit_threshold is not None:
            stats = self.get_early_exit_stats()
            if stats:
                print(format_early_exit_stats(self.early_exit_threshold, stats), end="")
        return prompt + "".join(pieces)
