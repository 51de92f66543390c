"""The step's plain fp16 GEMMs through qlora_gemm / qlora_gemm_splitk (rocBLAS, Tensile kernels)
and qlora_gemmlt (hipBLASLt) with a variant measured per weight shape and token-count bucket.

y = x W^T and dX = dY W (engine.py:1082-1316, 1376-1381) are torch matmuls in the reference,
i.e. whatever kernel the library's size heuristic picks. At this step's sizes (M = a few
thousand tokens) the heuristic leaves 20-40 % on the table: for the widest projections
(gate|up: 0.93 -> 1.15 PFLOP/s forward, 0.65 -> 0.83 backward on MI355X), and most for the
long-K, narrow-N input gradients (gate|up K = 17920, lm_head K = 151936, N = 1536), whose
output has too few tiles to fill 256 CUs - there a split of K into slices (fp32 partials, one
fixed-order sum) wins.

A variant is (solution, splits): solution -1 = torch's matmul, 0 = rocBLAS's own choice, > 0 a
Tensile solution index; splits 1 = one GEMM, > 1 = qlora_gemm_splitk; splits LT (0) =
qlora_gemmlt with hipBLASLt's first choice for the exact problem, whose epilogue adds a bias
before the one rounding (rocBLAS has no bias: the output is first filled with it, an extra
write and read of the output, +30 % on the qkv projection). The tuner times every solution
rocBLAS offers for a shape once (for each split count that divides K), keeps the fastest few as
candidates, and then, per bucket of BUCKET tokens, the fastest candidate, with the bias when the
shape has one. Every variant computes fp16(sum of fp16 products in fp32 (+ bias)); only the
summation order differs.

The package's own MFMA GEMM (qlora_hgemm: 256 x 256 tiles, bias or fp32-residual epilogue) is
one more candidate for the x W^T products whose reduction length it tiles (K % 128 == 0): it
wins where its one tile shape divides the work well (the [gate | up] product at 2,560 tokens:
139 against 155 us) and loses where its last round of tiles is nearly empty (2,561-2,816
tokens: 770 tiles on 256 CUs), which the per-bucket timing sorts out.

hipBLASLt's listed solutions are not candidates: they are mostly rocBLAS's own (rocBLAS runs
the same Tensile library on this GPU), none was faster than rocBLAS's best by more than 4 % at
the step's shapes with cold caches, and listing them costs ~30 ms of host time per new token
count and shape, against ~10 us for the first choice.
"""

import ctypes
import time

import torch

from . import _lib
from .ops import _need, _ptr, _resid_add, _stream

BUCKET = 256
TORCH = (-1, 1)   # torch's matmul
DEFAULT = (0, 1)  # rocBLAS's own choice
NT, NN = 0, 1     # op: C = A B^T (B [N, K]) or C = A B (B [K, N])
LT = 0           # splits value of the hipBLASLt variant
LT_DEFAULT = (0, LT)
PKG = (-2, 1)     # qlora_hgemm, the package's MFMA GEMM (op NT)
LT_WORKSPACE = 32 * 2**20  # bytes of workspace offered to hipBLASLt
SPLITS = (2, 4, 8)
MIN_SLICE = 1024  # no split leaves less than this much K per slice

_CANDIDATES = {}  # (device index, op, N, K, bias) -> [variant, ...]
_CHOICE = {}      # (device index, op, N, K, bias, bucket) -> variant


def _bucket(M):
    return -(-M // BUCKET)


def _dims(a, b, op):
    M, K = a.shape
    if op == NT:
        N, Kb = b.shape
    else:
        Kb, N = b.shape
    if Kb != K:
        raise ValueError(f"inner dimensions differ: {K} vs {Kb}")
    return M, N, K


def _check(t, name, dev):
    _need(t, name, torch.float16, dev, contiguous=False)
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a 2-D fp16 tensor with unit column stride")
    return t.stride(0)


def split_counts(N, K):
    """The split counts qlora_gemm_splitk accepts for this shape and the tuner tries."""
    if N % 4:
        return []
    return [s for s in SPLITS if K % (8 * s) == 0 and K // s >= MIN_SLICE]


def choice(dev_index, op, N, K, M, bias=False):
    """The variant used for this problem: the tuned one for M's bucket, else the nearest tuned
    bucket's, else torch's matmul."""
    b = _bucket(M)
    shape = (dev_index, op, N, K, bool(bias))
    v = _CHOICE.get(shape + (b,))
    if v is not None:
        return v
    near = [k[5] for k in _CHOICE if k[:5] == shape]
    if not near:
        return TORCH
    nb = min(near, key=lambda x: (abs(x - b), x))
    return _CHOICE[shape + (nb,)]


def pkg_fits(op, N, K):
    """Whether qlora_hgemm takes this product shape as a tuner candidate."""
    return op == NT and K % 128 == 0 and N % 8 == 0


def _run(variant, op, a, b, out, bias, M, N, K, lda, ldb, ldc, dev, work=None):
    sol, splits = variant
    if variant == PKG:
        _lib.call("qlora_hgemm", _ptr(a), lda, _ptr(b), ldb, M, N, K, op, _ptr(out), ldc,
                  _ptr(bias), None, 0, 1 if bias is not None else 0, 0, 1, None, 0,
                  _stream(dev))
        return
    if splits == LT:
        if work is None or work.numel() * work.element_size() < LT_WORKSPACE:
            work = torch.empty((LT_WORKSPACE,), device=dev, dtype=torch.uint8)
        _lib.call("qlora_gemmlt", op, M, N, K, _ptr(a), lda, _ptr(b), ldb, _ptr(out), ldc,
                  _ptr(bias), 1.0, 0.0, int(sol), _ptr(work), LT_WORKSPACE, _stream(dev))
        return
    if splits == 1:
        beta = 0.0
        if bias is not None:
            out.copy_(bias.view(1, N).expand(M, N))
            beta = 1.0
        _lib.call("qlora_gemm", op, M, N, K, _ptr(a), lda, _ptr(b), ldb, _ptr(out), ldc, 1.0,
                  beta, int(sol), _stream(dev))
        return
    if work is None:
        work = torch.empty((splits * M * N,), device=dev, dtype=torch.float32)
    _lib.call("qlora_gemm_splitk", op, M, N, K, _ptr(a), lda, _ptr(b), ldb, _ptr(out), ldc,
              _ptr(bias), splits, _ptr(work), work.numel(), int(sol), _stream(dev))


def mm(a, b, op, out=None, bias=None):
    """fp16 [M, N] = a b^T (op NT, b [N, K]) or a b (op NN, b [K, N]) [+ bias, one rounding];
    a, b, out with unit column stride."""
    dev = a.device
    lda = _check(a, "a", dev)
    ldb = _check(b, "b", dev)
    M, N, K = _dims(a, b, op)
    if out is None:
        out = torch.empty((M, N), device=dev, dtype=torch.float16)
    ldc = _check(out, "out", dev)
    if out.shape != (M, N):
        raise ValueError(f"out must be [{M}, {N}]")
    if bias is not None:
        _need(bias, "bias", torch.float16, dev)
        if bias.numel() != N:
            raise ValueError("bias must have one entry per output column")
    if M == 0:
        return out
    v = choice(dev.index or 0, op, N, K, M, bias is not None)
    if v == TORCH:
        bt = b.t() if op == NT else b
        if bias is not None:
            return torch.addmm(bias, a, bt, out=out)
        return torch.mm(a, bt, out=out)
    if v[1] > 1 and (ldc % 4 or out.data_ptr() % 8):
        v = DEFAULT
    try:
        _run(v, op, a, b, out, bias, M, N, K, lda, ldb, ldc, dev)
    except RuntimeError:
        if v == DEFAULT:
            raise
        # the bucket's variant rejects this exact size (the libraries check before launching);
        # the package's GEMM rejects operands by their alignment, so its choice stays
        if v != PKG:
            _CHOICE[(dev.index or 0, op, N, K, bias is not None, _bucket(M))] = DEFAULT
        _run(DEFAULT, op, a, b, out, bias, M, N, K, lda, ldb, ldc, dev)
    return out


def mm_resid(a, b, op, resid, out=None):
    """fp32 [M, N] = resid + fp32(fp16(a op(b))): the product rounded to fp16 as mm() rounds it,
    added to the fp32 residual stream (out may be resid). When the variant tuned for the product
    is a split of K, the split's reduce kernel adds the residual itself (no fp16 [M, N] output,
    no second pass); otherwise mm() and the residual-add kernel."""
    dev = a.device
    lda = _check(a, "a", dev)
    ldb = _check(b, "b", dev)
    M, N, K = _dims(a, b, op)
    _need(resid, "resid", torch.float32, dev, contiguous=False)
    if resid.shape != (M, N) or resid.stride(1) != 1:
        raise ValueError(f"resid must be [{M}, {N}] with unit column stride")
    if out is None:
        out = torch.empty((M, N), device=dev, dtype=torch.float32)
    _need(out, "out", torch.float32, dev, contiguous=False)
    if out.shape != (M, N) or out.stride(1) != 1:
        raise ValueError(f"out must be [{M}, {N}] with unit column stride")
    if M == 0:
        return out
    v = choice(dev.index or 0, op, N, K, M, False)
    sol, splits = v
    ldr, ldo = resid.stride(0), out.stride(0)
    if v == PKG:  # the residual added in the GEMM's epilogue
        try:
            _lib.call("qlora_hgemm", _ptr(a), lda, _ptr(b), ldb, M, N, K, op, _ptr(out), ldo,
                      None, _ptr(resid), ldr, 2, 0, 1, None, 0, _stream(dev))
            return out
        except RuntimeError:
            pass  # this exact problem is not tiled (alignment): the two-pass form below
    if sol >= 0 and splits > 1 and ldr % 4 == 0 and ldo % 4 == 0 and \
            resid.data_ptr() % 16 == 0 and out.data_ptr() % 16 == 0:
        work = torch.empty((splits * M * N,), device=dev, dtype=torch.float32)
        try:
            _lib.call("qlora_gemm_splitk_resid", op, M, N, K, _ptr(a), lda, _ptr(b), ldb,
                      _ptr(resid), ldr, _ptr(out), ldo, splits, _ptr(work), work.numel(),
                      int(sol), _stream(dev))
            return out
        except RuntimeError:
            pass  # the variant rejects this exact size: the two-pass form below
    return _resid_add(resid, mm(a, b, op), out=out)


def _listed(fn, *args):
    cnt = ctypes.c_int32(0)
    _lib.call(fn, *args, None, 0, ctypes.byref(cnt))
    if cnt.value == 0:
        return []
    arr = (ctypes.c_int32 * cnt.value)()
    _lib.call(fn, *args, arr, cnt.value, ctypes.byref(cnt))
    return list(arr)[:cnt.value]


def solutions(op, a, b, out, splits=1, work=None):
    """Every rocBLAS solution index for this problem (and split count; work: the fp32
    workspace of the split problem)."""
    dev = a.device
    lda, ldb = _check(a, "a", dev), _check(b, "b", dev)
    M, N, K = _dims(a, b, op)
    if splits == 1:
        ldc = _check(out, "out", dev)
        return _listed("qlora_gemm_solutions", op, M, N, K, _ptr(a), lda, _ptr(b), ldb,
                       _ptr(out), ldc)
    return _listed("qlora_gemm_splitk_solutions", op, M, N, K, _ptr(a), lda, _ptr(b), ldb,
                   _ptr(work), splits)


FLUSH_BYTES = 512 * 2**20  # > the 256 MB last-level (Infinity) cache of an MI355X
_FLUSH = {}


def _time(fn, reps):
    """Mean duration (ms) of fn over reps runs, each after the last-level cache was overwritten:
    in the step the operands come from HBM, and timing a variant against warm operands favours
    those that move more bytes (split-K's fp32 partials)."""
    fn()
    dev = torch.cuda.current_device()
    buf = _FLUSH.get(dev)
    if buf is None:
        buf = _FLUSH[dev] = torch.empty((FLUSH_BYTES // 4,), device=dev, dtype=torch.float32)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(reps)]
    for s, e in ev:
        buf.fill_(0.0)
        s.record()
        fn()
        e.record()
    ev[-1][1].synchronize()
    return sum(s.elapsed_time(e) for s, e in ev) / reps


def tune(shapes, Ms, device, top=6, top_split=2, reps=3, log=None):
    """Measure, for each (op, N, K[, bias]) in shapes and each token count in Ms, the fastest of:
    torch's matmul, rocBLAS's default, hipBLASLt's first choice, the package's GEMM (NT shapes
    it tiles), the `top` rocBLAS solutions that were fastest at the median token count and, per
    split count, rocBLAS's default and the `top_split` fastest; with a bias added when the shape
    has one. Buckets already tuned are skipped. Returns the seconds spent."""
    t0 = time.perf_counter()
    dev = torch.device(device)
    di = dev.index or 0
    buckets = sorted({_bucket(M) for M in Ms if M > 0})
    work = []
    for shape in shapes:
        op, N, K = shape[:3]
        has_bias = bool(shape[3]) if len(shape) > 3 else False
        todo = [bk for bk in buckets if (di, op, N, K, has_bias, bk) not in _CHOICE]
        if todo:
            work.append((op, N, K, has_bias, todo))
    if not work:
        return 0.0
    m_max = buckets[-1] * BUCKET
    g = torch.Generator(device=dev).manual_seed(0)
    for op, N, K, has_bias, todo in work:
        a_full = torch.randn((m_max, K), device=dev, generator=g).to(torch.float16)
        bshape = (N, K) if op == NT else (K, N)
        b = (torch.randn(bshape, device=dev, generator=g) * 0.02).to(torch.float16)
        bias = (torch.randn((N,), device=dev, generator=g) * 0.02).to(torch.float16) \
            if has_bias else None
        c_full = torch.empty((m_max, N), device=dev, dtype=torch.float16)
        splits_ok = split_counts(N, K)
        ws = torch.empty((max(splits_ok, default=0) * m_max * N or 1,), device=dev,
                         dtype=torch.float32)
        lt_ws = torch.empty((LT_WORKSPACE,), device=dev, dtype=torch.uint8)
        ldb = b.stride(0)

        def runner(v, M):
            a, c = a_full[:M], c_full[:M]
            if v == TORCH:
                bt = b.t() if op == NT else b
                if bias is not None:
                    return lambda: torch.addmm(bias, a, bt, out=c)
                return lambda: torch.mm(a, bt, out=c)
            w = lt_ws if v[1] == LT else ws
            return lambda: _run(v, op, a, b, c, bias, M, N, K, K, ldb, N, dev, work=w)

        def listed(M, splits):
            return solutions(op, a_full[:M], b, c_full[:M], splits, ws)

        key = (di, op, N, K, has_bias)
        if key not in _CANDIDATES:
            m_mid = todo[len(todo) // 2] * BUCKET
            cands = [TORCH, DEFAULT, LT_DEFAULT] + ([PKG] if pkg_fits(op, N, K) else [])
            for splits, keep in [(1, top)] + [(s, top_split) for s in splits_ok]:
                timed = []
                for sol in listed(m_mid, splits):
                    try:
                        timed.append((_time(runner((sol, splits), m_mid), 1), sol))
                    except RuntimeError:
                        continue  # a solution that rejects the problem is not a candidate
                timed.sort()
                if splits > 1:
                    cands.append((0, splits))
                cands += [(s, splits) for _, s in timed[:keep] if s != 0]
            _CANDIDATES[key] = cands
        for bk in todo:
            M = bk * BUCKET
            valid = {TORCH, DEFAULT, LT_DEFAULT, PKG}
            for splits in [1] + splits_ok:
                valid |= {(s, splits) for s in [0] + listed(M, splits)}
            timed = []
            for v in _CANDIDATES[key]:
                if v not in valid:
                    continue
                try:
                    timed.append((_time(runner(v, M), reps), v))
                except RuntimeError:
                    continue  # e.g. hipBLASLt has no solution for this problem
            best = min(timed)
            _CHOICE[key + (bk,)] = best[1]
            if log is not None:
                log(f"gemm tune op={op} N={N} K={K} bias={int(has_bias)} M={M}: {best[1]} "
                    f"{best[0] * 1e3:.1f} us")
        del a_full, b, c_full, ws, lt_ws, bias
    return time.perf_counter() - t0


def reset():
    """Forget every measurement and the flush buffers (tests)."""
    _CANDIDATES.clear()
    _CHOICE.clear()
    _FLUSH.clear()
