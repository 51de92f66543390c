"""The kernel-call layer: the reference engine's op wrappers, same names, signatures and argument
meaning (solution/engine.py:683-1045), each launching one gfx950 kernel of libqlora_amd.so on
torch's current HIP stream.

Ownership as in the reference: wrappers allocate their outputs with torch.empty on the input's
device; `_glu_bwd` overwrites `gu`, `_ce` the logits, `_ce_piece` the logits rows below n_sup and
its state tensors. Inputs are checked (device, dtype, shape, contiguity) before any launch, and a
CPU tensor is refused: there is no CPU path.
"""

import ctypes
import itertools

import torch

from . import _lib

# launch-shape constants of the reference that are part of the interface (engine.py:42-47)
CE_BLOCK = 4096  # (the reference's vocabulary block; pieces must start on a multiple of it)
HEAD_CHUNK = 256
PIECE = 8192  # vocabulary rows per piece of the chunked head (engine.py:1414)


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream(device):
    """torch's current HIP stream on `device` (raw handle, as the C-ABI takes it)."""
    return torch._C._cuda_getCurrentRawStream(
        device.index if device.index is not None else torch.cuda.current_device())


def _need(t, name, dtype=None, device=None, contiguous=True):
    if t is None:
        raise ValueError(f"{name} is required")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor (got {t.device}); there is no CPU path")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype} (got {t.dtype})")
    if contiguous and not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


def _rows_view(t, name, dtype, rows, cols, device):
    """A [rows, cols] tensor with unit column stride; returns its row stride."""
    _need(t, name, dtype, device, contiguous=False)
    if t.dim() != 2 or t.shape[0] != rows or t.shape[1] != cols or t.stride(1) != 1:
        raise ValueError(f"{name} must be [{rows}, {cols}] with unit column stride")
    return t.stride(0)


# ---------------------------------------------------------------------------------------------
# NF4 weights in bitsandbytes' storage (read in place; the reference's wrappers read the same
# Params4bit fields, engine.py:74-157, and stack weights the same way, 683-694)
# ---------------------------------------------------------------------------------------------
NF4_LEVELS = (-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
              -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
              0.07958029955625534, 0.16093020141124725, 0.24611230194568634,
              0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
              0.7229568362236023, 1.0)
_NO_SEG = 2**63 - 1  # a segment bound past every block: "no further segment"


def _f32(t):
    return t.detach().to(torch.float32).contiguous()


def _is_nf4_table(code):
    """Whether a 16-entry code is bitsandbytes' NF4 table (the kernels then use their own copy
    of it instead of loading the code)."""
    if code.numel() != 16:
        return False
    ref = torch.tensor(NF4_LEVELS, dtype=torch.float32, device=code.device)
    return bool((code.reshape(-1) == ref).all())


def _offset_tensor(offset, device):
    if torch.is_tensor(offset):
        return offset.detach().to(device=device, dtype=torch.float32).reshape(1).clone()
    return torch.tensor([float(offset)], device=device, dtype=torch.float32)


class NF4Weight:
    """A frozen Linear4bit weight [N, K] as bitsandbytes stores it, read without a copy.

    `param.data` holds the codes, two per byte (element 2j in the high nibble of byte j);
    `param.quant_state` holds one scale per `bs1` consecutive elements. With double
    quantisation (`nested`) each scale is itself an 8-bit code: scale = code2[absmax[b]] *
    absmax2[b // bs2] + offset; otherwise `absmax` is the fp32 scale. The attributes below are
    what the dequant and fused-GEMM entry points take."""

    def __init__(self, param):
        st = param.quant_state
        rows, cols = (int(d) for d in st.shape)
        dev = param.data.device
        self.param, self.packed, self.group = param, param.data, None
        self.shape, self.numel = (rows, cols), rows * cols
        self.bs1 = int(st.blocksize)
        if self.numel % self.bs1:
            raise ValueError(f"a {rows} x {cols} weight does not split into blocks of "
                             f"{self.bs1} values")
        self.code = _f32(st.code)
        self.standard = _is_nf4_table(self.code)
        self.nested = bool(getattr(st, "nested", False))
        if self.nested:
            inner = st.state2
            self.bs2 = int(inner.blocksize)
            self.absmax = st.absmax  # uint8 codes into code2
            self.code2, self.absmax2 = _f32(inner.code), _f32(inner.absmax)
            self.offset = _offset_tensor(st.offset, dev)
        else:
            self.bs2 = 1
            self.absmax = _f32(st.absmax)  # the scales themselves
            self.code2 = self.absmax2 = self.offset = None
        self._args = _dequant_args(self.packed, self.absmax, self.code2, self.absmax2,
                                   self.offset, self.code, self.blocks, self.nested,
                                   self.standard, self.bs1, self.bs2, _NO_SEG, _NO_SEG,
                                   self.numel)
        self._scales = None

    def block_scales(self):
        """fp32 [blocks]: each block's scale, the operand of the fused NF4 GEMM."""
        if self._scales is None:
            self._scales = _block_scales(self, self.offset, _NO_SEG, _NO_SEG)
        return self._scales

    @property
    def blocks(self):
        return self.numel // self.bs1

    @property
    def layout(self):
        """What two weights must share to be decoded by one launch over their concatenation:
        row length, block sizes, double quantisation and the code table."""
        return (self.shape[1], self.bs1, self.bs2, self.nested, self.standard)

    def dequant_into(self, out):
        _launch_dequant(self._args, out, self.blocks, self.nested, self.standard, self.bs1,
                        self.bs2, _NO_SEG, _NO_SEG, self.numel, self.packed.device)
        return out


def _same_tables(a, b):
    if not torch.equal(a.code, b.code):
        return False
    return not a.nested or torch.equal(a.code2, b.code2)


class NF4Group:
    """2 or 3 NF4 weights with the same layout, concatenated along their rows (q|k|v, gate|up)
    so that one launch decodes all of them. The packed codes and absmax are concatenated into
    resident copies; with double quantisation the per-weight offsets become segments: block b
    takes offsets[0] below seg1, offsets[1] below seg2, offsets[2] after that. Concatenating the
    absmax2 tables keeps block b's entry at b // bs2 only if every weight but the last covers
    whole bs2-block groups."""

    @classmethod
    def of(cls, weights):
        """The group of these weights, or None when they cannot share one launch."""
        weights = list(weights)
        if len(weights) not in (2, 3):
            return None
        first = weights[0]
        if any(w.layout != first.layout or not _same_tables(w, first) for w in weights[1:]):
            return None
        if any(w.blocks % w.bs2 for w in weights[:-1]):
            return None
        return cls(weights)

    def __init__(self, weights):
        first = weights[0]
        self.weights = list(weights)
        self.nested, self.standard = first.nested, first.standard
        self.bs1, self.bs2 = first.bs1, first.bs2
        self.code, self.code2 = first.code, first.code2
        ends = list(itertools.accumulate(w.blocks for w in self.weights))
        self.blocks = ends[-1]
        self.numel = self.blocks * self.bs1
        self.seg1, self.seg2 = (ends[:-1] + [_NO_SEG, _NO_SEG])[:2]
        self.packed = torch.cat([w.packed.reshape(-1) for w in self.weights])
        self.absmax = torch.cat([w.absmax.reshape(-1) for w in self.weights])
        if self.nested:
            self.absmax2 = torch.cat([w.absmax2.reshape(-1) for w in self.weights])
            self.offsets = torch.cat([w.offset for w in self.weights])
        else:
            self.absmax2 = self.offsets = None
        for w in self.weights:
            w.group = self
        self._args = _dequant_args(self.packed, self.absmax, self.code2, self.absmax2,
                                   self.offsets, self.code, self.blocks, self.nested,
                                   self.standard, self.bs1, self.bs2, self.seg1, self.seg2,
                                   self.numel)
        self._scales = None

    def block_scales(self):
        """fp32 [blocks]: each block's scale (its weight's offset by segment)."""
        if self._scales is None:
            self._scales = _block_scales(self, self.offsets, self.seg1, self.seg2)
        return self._scales

    @property
    def shape(self):
        return sum(w.shape[0] for w in self.weights), self.weights[0].shape[1]

    def dequant_into(self, out):
        _launch_dequant(self._args, out, self.blocks, self.nested, self.standard, self.bs1,
                        self.bs2, self.seg1, self.seg2, self.numel, self.packed.device)
        return out


def _dequant_args(packed, absmax, code2, absmax2, offsets, code, blocks, nested, standard, bs1,
                  bs2, seg1, seg2, numel):
    """Checks a weight's quantization state once and returns the qlora_nf4_dequant arguments
    that do not change between launches (everything but the output and the stream)."""
    dev = packed.device
    _need(packed, "packed", torch.uint8, dev, contiguous=False)
    if packed.numel() * 2 != numel or not packed.is_contiguous():
        raise ValueError("packed must hold numel / 2 contiguous bytes")
    _need(absmax, "absmax", torch.uint8 if nested else torch.float32, dev)
    if absmax.numel() != blocks:
        raise ValueError("absmax must have one entry per block")
    if nested:
        _need(code2, "code2", torch.float32, dev)
        _need(absmax2, "absmax2", torch.float32, dev)
        _need(offsets, "offsets", torch.float32, dev)
        if code2.numel() != 256 or absmax2.numel() < (blocks + bs2 - 1) // bs2:
            raise ValueError("code2 must have 256 entries and absmax2 one per block of absmax")
    if not standard:
        _need(code, "code", torch.float32, dev)
        if code.numel() != 16:
            raise ValueError("code must have 16 entries")
    return (_ptr(packed), _ptr(absmax), _ptr(code2) if nested else None,
            _ptr(absmax2) if nested else None, _ptr(offsets) if nested else None, _ptr(code))


def _launch_dequant(args, out, blocks, nested, standard, bs1, bs2, seg1, seg2, numel, dev):
    if out.dtype != torch.float16 or out.device != dev or not out.is_contiguous() \
            or out.numel() != numel:
        raise ValueError(f"out must be a contiguous fp16 tensor of {numel} elements on {dev}")
    if blocks == 0:
        return
    _lib.call("qlora_nf4_dequant", *args, _ptr(out), blocks, int(nested), int(standard), bs1,
              bs2, seg1, seg2, _stream(dev))


def _block_scales(w, offsets, seg1, seg2):
    """The fp32 scale of each block of an NF4Weight / NF4Group (qlora_nf4_block_scales): the
    absmax itself without double quantisation, else decoded once - the weights are frozen, so
    the fused GEMM reads one word per block for the whole run."""
    if not w.nested:
        return w.absmax
    out = torch.empty(w.blocks, device=w.packed.device, dtype=torch.float32)
    _lib.call("qlora_nf4_block_scales", _ptr(w.absmax), _ptr(w.code2), _ptr(w.absmax2),
              _ptr(offsets), 1, w.bs2, seg1, seg2, w.blocks, _ptr(out),
              _stream(w.packed.device))
    return out


GEMM_TILE = 256  # W rows per tile of the fused GEMM (qlora_nf4_gemm)


def _gemm_tile_rows(w_rows, swiglu_I):
    """The W row each position of the tile-major order holds (qlora_nf4_gemm, tiled): tile t's
    row r is W row 256 t + r, or with the SwiGLU epilogue row j = 128 t + 64 (r // 128) + r % 64
    of the gate (r % 128 < 64) or the up projection (I + j)."""
    n = torch.arange(w_rows, dtype=torch.int64)
    if not swiglu_I:
        return n
    t, r = n // GEMM_TILE, n % GEMM_TILE
    j = t * 128 + (r // 128) * 64 + r % 64
    return torch.where(r % 128 >= 64, swiglu_I + j, j)


def gemm_tiles(w, swiglu_I=0):
    """The codes and fp32 block scales of an NF4Weight / NF4Group in the fused GEMM's tile-major
    order for y = x W^T (qlora_nf4_gemm, tiled = 1): formed once per weight and layout (the
    weights are frozen) and kept on it; the same bytes as the bitsandbytes order, rearranged so
    that each k-tile of a 256-row tile is 4 KB of codes and 1 KB of scales in a row."""
    cache = w.__dict__.setdefault("_gemm_tiles", {})
    if swiglu_I in cache:
        return cache[swiglu_I]
    rows, cols = w.shape
    if rows % GEMM_TILE or cols % 64 or w.bs1 != 64:
        raise ValueError("the tile-major order takes 256-row tiles of 64-value blocks")
    if swiglu_I and 2 * swiglu_I != rows:
        raise ValueError("the SwiGLU order takes [gate; up] with I rows each")
    dev = w.packed.device
    order = _gemm_tile_rows(rows, swiglu_I).to(dev)
    tiles, kt = rows // GEMM_TILE, cols // 32
    codes = w.packed.reshape(rows, cols // 2).index_select(0, order)
    codes = codes.view(tiles, GEMM_TILE, kt, 16).permute(0, 2, 1, 3).contiguous().view(-1)
    scales = w.block_scales().reshape(rows, cols // 64).index_select(0, order)
    scales = scales.view(tiles, GEMM_TILE, cols // 64).permute(0, 2, 1).contiguous().view(-1)
    cache[swiglu_I] = (codes, scales)
    return cache[swiglu_I]


def _dq_segs(w):
    return (w.seg1, w.seg2) if isinstance(w, NF4Group) else (_NO_SEG, _NO_SEG)


DEQUANT_MANY_MAX = 32  # weights per qlora_nf4_dequant_many launch


def dequant_many(items, device, outs=None):
    """fp16 [N_i, K_i] of each NF4Weight / NF4Group of `items` (at most DEQUANT_MANY_MAX), all
    in one launch (a layer's qkv, o, gate|up and down, or those of several layers). `outs`:
    contiguous fp16 destinations of the right sizes, else they are allocated."""
    if not 1 <= len(items) <= DEQUANT_MANY_MAX:
        raise ValueError(f"dequant_many takes 1 to {DEQUANT_MANY_MAX} weights")
    if outs is None:
        outs = [torch.empty(w.shape, device=device, dtype=torch.float16) for w in items]
    if len(outs) != len(items):
        raise ValueError("one output per weight")
    device = outs[0].device  # "cuda" -> "cuda:<current>"
    for w, o in zip(items, outs):
        if w.packed.device != device:
            raise ValueError(f"weight on {w.packed.device}, expected {device}")
        _need(o, "out", torch.float16, device)
        if o.numel() != w.numel:
            raise ValueError(f"out has {o.numel()} elements, the weight {w.numel}")
    k = len(items)
    P = ctypes.c_void_p * k
    args = [P(*[w._args[i] for w in items]) for i in range(6)]
    segs = [_dq_segs(w) for w in items]
    _lib.call("qlora_nf4_dequant_many", k, *args, P(*[o.data_ptr() for o in outs]),
              (ctypes.c_int64 * k)(*[w.blocks for w in items]),
              (ctypes.c_int32 * k)(*[int(w.nested) for w in items]),
              (ctypes.c_int32 * k)(*[int(w.standard) for w in items]),
              (ctypes.c_int32 * k)(*[w.bs1 for w in items]),
              (ctypes.c_int32 * k)(*[w.bs2 for w in items]),
              (ctypes.c_int64 * k)(*[s[0] for s in segs]),
              (ctypes.c_int64 * k)(*[s[1] for s in segs]), _stream(device))
    return outs


def dequant(weights, device):
    """fp16 [sum N_i, K]: the weights decoded one below the other (engine.py:683-694's
    contract). One launch either way: the group's own when the weights are exactly a group,
    else one qlora_nf4_dequant_many launch writing each weight's row range."""
    weights = list(weights)
    cols = {w.shape[1] for w in weights}
    if len(cols) != 1:
        raise ValueError("stacked weights must have the same number of columns")
    rows = [w.shape[0] for w in weights]
    out = torch.empty((sum(rows), cols.pop()), device=device, dtype=torch.float16)
    group = weights[0].group
    if group is not None and group.weights == weights:
        return group.dequant_into(out)
    bounds = [0, *itertools.accumulate(rows)]
    for i in range(0, len(weights), DEQUANT_MANY_MAX):
        part = weights[i:i + DEQUANT_MANY_MAX]
        dequant_many(part, out.device,
                     outs=[out[bounds[j]:bounds[j + 1]] for j in range(i, i + len(part))])
    return out


# ---------------------------------------------------------------------------------------------
# LoRA dropout masks: the Philox stream of PyTorch's dropout (engine.py:767-828 draws from the
# same generator; the mask arithmetic is kernels.py:108-135's, restated for rocRAND)
# ---------------------------------------------------------------------------------------------
def _as_int64(x):
    """A 64-bit seed as the signed value the C-ABI takes (same bits)."""
    return x - 2**64 if x >= 2**63 else x


class TorchDropout:
    """Where the masks of PEFT's LoRA dropout come from, so that the kernels can recompute them.

    PEFT applies nn.Dropout(p) to each adapter's input, a contiguous [B, T, H] tensor, in the
    order the forward reaches the adapters (layer 0 q, layer 0 v, layer 1 q, ...). On ROCm that
    dropout is one fused launch of up to `max_blocks` blocks of 256 threads (the device's CUs x
    the blocks resident per CU); thread i of the grid draws Philox4x32-10 outputs at counter
    (offset/4 + round, i) of the default generator, four values a round and `vec` elements per
    16-byte access, and the launch moves the generator's offset past the rounds it used.
    `draw` hands out the (seed, counter, threads) of the next such call and moves the generator
    exactly as that launch would; `check` compares the RMSNorm kernel's mask with nn.Dropout's
    own on this device, once."""

    THREADS_PER_BLOCK = 256
    VALUES_PER_ROUND = 4

    CHECK_SEED = 0x1D20_2F5B  # seeds the self-check's private generator state
    CHECK_TOKENS = 48         # tokens per row checked

    def __init__(self, device, dtype):
        self.device = torch.device(device)
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.dtype = dtype
        props = torch.cuda.get_device_properties(self.device)
        self.max_blocks = props.multi_processor_count * (
            props.max_threads_per_multi_processor // self.THREADS_PER_BLOCK)
        self.gen = torch.cuda.default_generators[self.device.index]
        self.vec = 16 // torch.empty((), dtype=dtype).element_size()
        if self.vec not in (4, 8):
            raise ValueError(f"dropout input dtype {dtype} is not 2 or 4 bytes wide")
        self.ok = None  # the self-check's verdict, once run

    def launch(self, nelem):
        """(threads, counter advance) of PyTorch's dropout launch over nelem elements."""
        blocks = max(1, min(self.max_blocks, -(-nelem // self.THREADS_PER_BLOCK)))
        threads = blocks * self.THREADS_PER_BLOCK
        rounds = -(-nelem // (threads * self.VALUES_PER_ROUND))
        return threads, rounds * self.VALUES_PER_ROUND

    def draw(self, nelem):
        """(seed, counter, threads) of the next dropout call on nelem elements; the generator
        moves on as that call would move it."""
        if nelem % self.vec:
            raise ValueError(f"{nelem} elements are not whole {self.vec}-element accesses")
        threads, advance = self.launch(nelem)
        seed, offset = self.gen.initial_seed(), self.gen.get_offset()
        self.gen.set_offset(offset + advance)
        return _as_int64(seed), offset // 4, threads

    def check(self, B, T, H, p):
        """True when the RMSNorm kernel's q mask equals nn.Dropout's on this device: F.dropout
        of ones over [B, T, H] and our mask drawn from the same freshly seeded generator state,
        inside a fork of the RNG state (the caller's generator is left where it was)."""
        with torch.random.fork_rng(devices=[self.device.index], device_type="cuda"):
            self.gen.manual_seed(self.CHECK_SEED)
            ones = torch.ones((B, T, H), device=self.device, dtype=self.dtype)
            want = torch.nn.functional.dropout(ones, p=p, training=True) != 0
            self.gen.manual_seed(self.CHECK_SEED)
            seed, ctr, threads = self.draw(B * T * H)

        class _Rows:  # the fields _rms_fwd reads from a spec and a packed batch
            eps = 1e-6
            dropout_p, drop_seed, drop_threads, drop_vec = p, seed, threads, self.vec
            tok = torch.arange(B * T, device=self.device)

        x = torch.ones((B * T, H), device=self.device, dtype=torch.float32)
        _, _, got, _, _ = _rms_fwd(_Rows, x, torch.ones(H, device=self.device), _Rows,
                                   write_y=False, seeds=(ctr, 0), drop_q=True)
        return bool(torch.equal(got.view(B, T, H) != 0, want))


def keep_mask(nelem, seed, ctr, threads, p, vec, device):
    """Keep mask (bool [nelem]) of one dropout call (the test hook, kernels.py:129-135)."""
    out = torch.empty(nelem, device=device, dtype=torch.int8)
    _lib.call("qlora_dropout_keep", _ptr(out), nelem, int(seed), int(ctr), int(threads),
              1.0 - p, int(vec), _stream(out.device))
    return out.bool()


# ---------------------------------------------------------------------------------------------
# RMSNorm + LoRA dropout (engine.py:933-981)
# ---------------------------------------------------------------------------------------------
_DUMMIES = {}


def _dropout_args(packed, x, seeds):
    """The rms kernels' dropout arguments (engine.py:933-941): the tokens' indices in the padded
    batch, the keep probability and scale, the generator's seed, the q and v counters, threads."""
    tok = getattr(packed, "tok", None)
    p = getattr(packed, "dropout_p", 0.0) or 0.0
    rows, T = getattr(packed, "rows", 0), getattr(packed, "T", 0)
    if rows * T * x.shape[1] >= 2**32:
        raise ValueError("the dropout element index (token * H + column) must stay below 2^32")
    return (tok, 1.0 - p, 1.0 / (1.0 - p), getattr(packed, "drop_seed", None) or 0, seeds[0],
            seeds[1], getattr(packed, "drop_threads", None) or 1)


def _weight_arg(weight, H, device):
    _need(weight, "weight", None, device)
    if weight.dtype not in (torch.float32, torch.float16) or weight.numel() != H:
        raise ValueError("norm weight must be fp32 or fp16 with H entries")
    return int(weight.dtype == torch.float16)


def keep_bits_shape(n, H):
    """Shape of the keep-bit buffer of _rms_fwd / _rms_bwd (uint8): two masks (q, v) per row,
    bit k of byte j = element 4 j + k kept."""
    return (n, 2, (H + 3) // 4)


def _keep_arg(keep, n, H, dev):
    if keep is None:
        return None
    _need(keep, "keep", torch.uint8, dev)
    if tuple(keep.shape) != keep_bits_shape(n, H):
        raise ValueError(f"keep must be uint8 {keep_bits_shape(n, H)}")
    return _ptr(keep)


def _ctr_base(packed, dev):
    """Device pointer of the step's first dropout counter when the batch keeps it on the device
    (its masks' counters are then relative to it), else None."""
    base = getattr(packed, "ctr_base", None)
    if base is None:
        return None
    _need(base, "packed.ctr_base", torch.int64, dev)
    if base.numel() != 1:
        raise ValueError("packed.ctr_base must hold one int64")
    return _ptr(base)


def _rms_fwd(spec, x, weight, packed, *, delta=None, write_y=True, seeds=(0, 0),
             drop_q=False, drop_v=False, keep=None, keep_in=None):
    """[x += delta] + RMSNorm -> (xsum, y fp16, yq, yv, rstd) (engine.py:947-966). With keep
    (uint8 keep_bits_shape(n, H)) the dropout masks are also stored there as bits, for
    _rms_bwd to read instead of drawing them again; with keep_in the masks are read from bits
    an earlier pass over the same rows stored (a recompute), not drawn."""
    _need(x, "x", torch.float32)
    n, H = x.shape
    dev = x.device
    w_half = _weight_arg(weight, H, dev)
    if delta is not None:
        _need(delta, "delta", torch.float16, dev)
        if delta.shape != x.shape:
            raise ValueError("delta must match x")
    xsum = torch.empty_like(x) if delta is not None else x
    y = torch.empty((n, H), device=dev, dtype=torch.float16) if write_y else None
    yq = torch.empty((n, H), device=dev, dtype=torch.float16) if drop_q else None
    yv = torch.empty((n, H), device=dev, dtype=torch.float16) if drop_v else None
    rstd = torch.empty((n,), device=dev, dtype=torch.float32)
    keep_p = _keep_arg(keep, n, H, dev)
    keep_in_p = _keep_arg(keep_in, n, H, dev)
    if keep_in_p is not None and (keep_p is not None or not (drop_q or drop_v)):
        raise ValueError("keep_in reads the masks of a dropping pass that stores none itself")
    if n:
        tok, p_keep, keep_scale, seed, ctr_q, ctr_v, threads = _dropout_args(packed, x, seeds)
        vec = getattr(packed, "drop_vec", 4)
        if drop_q or drop_v:
            _need(tok, "packed.tok", torch.int64, dev)
            if tok.numel() != n:
                raise ValueError("packed.tok must have one entry per row")
        _lib.call("qlora_rms_fwd", _ptr(x), _ptr(delta), _ptr(weight), w_half,
                  _ptr(xsum) if delta is not None else None, _ptr(y), _ptr(yq), _ptr(yv),
                  _ptr(rstd), _ptr(tok) if (drop_q or drop_v) else None, n, H,
                  float(spec.eps), p_keep, keep_scale, int(seed), int(ctr_q), int(ctr_v),
                  int(threads), int(delta is not None), int(write_y), int(drop_q), int(drop_v),
                  int(vec), keep_p, keep_in_p, _ctr_base(packed, dev), _stream(dev))
    return xsum, y, yq, yv, rstd


def _rms_bwd(spec, dy, x, rstd, weight, packed, *, dres=None, tq=None, tv=None, seeds=(0, 0),
             grad_scale=1.0, out=None, out16=None, keep=None, xdelta=None, dy_parts=None):
    """RMSNorm backward with the LoRA-dropout gradients merged (engine.py:969-981). With out16
    (fp16 [n, H]) the kernel also writes fp16(dx) there, the operand the next backward product
    rounds the gradient to. keep: the masks _rms_fwd stored for these rows (same packed and
    seeds), or None to draw them again. xdelta (fp16 [n, H]): the forward normed x + xdelta
    (_rms_fwd with delta); the kernel forms that sum and its rstd again, in the forward's order
    of operations (the same bits), and rstd is not read (may be None). dy_parts (fp32
    [S, n, H], no dropout): dy is fp16 of these split-K slices summed in order (a product's
    qlora_gemm16_parts output, its reduce done here); dy is then None."""
    _need(x, "x", torch.float32)
    n, H = x.shape
    dev = x.device
    w_half = _weight_arg(weight, H, dev)
    if dy_parts is not None:
        _need(dy_parts, "dy_parts", torch.float32, dev)
        if dy_parts.dim() != 3 or tuple(dy_parts.shape[1:]) != (n, H) or \
                not 1 <= dy_parts.shape[0] <= 16 or tq is not None or tv is not None:
            raise ValueError("dy_parts must be fp32 [S <= 16, n, H], without dropout inputs")
        dy_stride = H
    else:
        dy_stride = _rows_view(dy, "dy", torch.float16, n, H, dev) if n else H
    if xdelta is not None:
        _need(xdelta, "xdelta", torch.float16, dev)
        if xdelta.shape != x.shape:
            raise ValueError("xdelta must match x")
    else:
        _need(rstd, "rstd", torch.float32, dev)
    for t, name in ((tq, "tq"), (tv, "tv")):
        if t is not None:
            _need(t, name, torch.float16, dev)
            if t.shape != x.shape:
                raise ValueError(f"{name} must match x")
    if dres is not None:
        _need(dres, "dres", torch.float32, dev)
        if dres.shape != x.shape:
            raise ValueError("dres must match x")
    dx = out if out is not None else torch.empty_like(x)
    _need(dx, "out", torch.float32, dev)
    if out16 is not None:
        _need(out16, "out16", torch.float16, dev)
        if out16.shape != x.shape:
            raise ValueError("out16 must match x")
    keep_p = _keep_arg(keep, n, H, dev)
    if n:
        tok, p_keep, keep_scale, seed, ctr_q, ctr_v, threads = _dropout_args(packed, x, seeds)
        vec = getattr(packed, "drop_vec", 4)
        if tq is not None or tv is not None:
            _need(tok, "packed.tok", torch.int64, dev)
        _lib.call("qlora_rms_bwd", _ptr(dy), _ptr(tq), _ptr(tv), _ptr(x), _ptr(rstd),
                  _ptr(weight), w_half, _ptr(dres), _ptr(dx), _ptr(out16),
                  _ptr(tok) if (tq is not None or tv is not None) else None, n, H, dy_stride,
                  p_keep, keep_scale, int(seed), int(ctr_q), int(ctr_v), int(threads),
                  float(grad_scale), int(tq is not None), int(tv is not None),
                  int(dres is not None), int(vec), keep_p, _ctr_base(packed, dev),
                  _ptr(xdelta), float(spec.eps), _ptr(dy_parts),
                  0 if dy_parts is None else dy_parts.shape[0], _stream(dev))
    return dx


# ---------------------------------------------------------------------------------------------
# qkv + RoPE (engine.py:984-1009)
# ---------------------------------------------------------------------------------------------
def _rope_fwd(spec, qkv, lq, lv, packed, lora_scale, kv_heads=None):
    """(q, k, v) fp16 [n, heads, D] from the fused qkv GEMM output and the LoRA deltas
    (engine.py:984-997). k and v come out repeated for the GQA groups ([n, HQ, D]) as in the
    reference, or with kv_heads=spec.HKV in grouped layout."""
    HQ, HKV, D = spec.HQ, spec.HKV, spec.D
    C = (HQ + 2 * HKV) * D
    _need(qkv, "qkv", torch.float16)
    n = qkv.shape[0]
    dev = qkv.device
    if qkv.shape != (n, C):
        raise ValueError(f"qkv must be [n, {C}]")
    if lq is not None:
        _need(lq, "lq", torch.float16, dev)
        if lq.shape != (n, HQ * D):
            raise ValueError("lq must be [n, HQ*D]")
    if lv is not None:
        _need(lv, "lv", torch.float16, dev)
        if lv.shape != (n, HKV * D):
            raise ValueError("lv must be [n, HKV*D]")
    kh = HQ if kv_heads is None else int(kv_heads)
    q = torch.empty((n, HQ, D), device=dev, dtype=torch.float16)
    k = torch.empty((n, kh, D), device=dev, dtype=torch.float16)
    v = torch.empty((n, kh, D), device=dev, dtype=torch.float16)
    if n:
        cos, sin, pos = _rope_tables(packed, D, n, dev)
        _lib.call("qlora_rope_fwd", _ptr(qkv), _ptr(lq), _ptr(lv), _ptr(cos), _ptr(sin),
                  cos.shape[0], _ptr(pos), _ptr(q), _ptr(k), _ptr(v), n, HQ, HKV, D, kh,
                  float(lora_scale), _stream(dev))
    return q, k, v


def _rope_bwd(spec, dq, dk, dv, packed):
    """[dq | dk | dv] pre-rotary gradient of the fused qkv output (engine.py:1000-1009)."""
    HQ, HKV, D = spec.HQ, spec.HKV, spec.D
    n = dq.shape[0]
    dev = dq.device
    dq, dk, dv = dq.contiguous(), dk.contiguous(), dv.contiguous()
    _need(dq, "dq", torch.float16)
    kh = dk.shape[1]
    for t, name in ((dk, "dk"), (dv, "dv")):
        _need(t, name, torch.float16, dev)
        if t.shape != (n, kh, D):
            raise ValueError(f"{name} must be [n, heads, D]")
    if dq.shape != (n, HQ, D):
        raise ValueError("dq must be [n, HQ, D]")
    C = (HQ + 2 * HKV) * D
    dqkv = torch.empty((n, C), device=dev, dtype=torch.float16)
    if n:
        cos, sin, pos = _rope_tables(packed, D, n, dev)
        _lib.call("qlora_rope_bwd", _ptr(dq), _ptr(dk), _ptr(dv), _ptr(cos), _ptr(sin),
                  cos.shape[0], _ptr(pos), _ptr(dqkv), n, HQ, HKV, D, kh, _stream(dev))
    return dqkv


def _resid_add(a, d, out=None):
    """a + fp32(d) (fp32 residual stream plus an fp16 projection output; engine.py:1048-1051)."""
    _need(a, "a", torch.float32)
    _need(d, "d", torch.float16, a.device)
    if d.shape != a.shape:
        raise ValueError("d must match a")
    out = torch.empty_like(a) if out is None else out
    _need(out, "out", torch.float32, a.device)
    if out.shape != a.shape:
        raise ValueError("out must match a")
    n = a.numel()
    if n % 4:
        raise ValueError("numel must be a multiple of 4")
    if n:
        _lib.call("qlora_resid_add", _ptr(a), _ptr(d), _ptr(out), n, _stream(a.device))
    return out


# ---------------------------------------------------------------------------------------------
# LoRA per-token products (engine.py:1088-1093, 1319-1331)
# ---------------------------------------------------------------------------------------------
def _lora_fwd_rows(a_q, a_v, A_q, B_q, A_v, B_v, need_l=True):
    """(x_q, x_v, l_q, l_v): x = fp16(a A^T) [n, r], l = fp16(x B^T) [n, N] for the q and v
    adapters (engine.py:1088-1093); a [n, H], A [r, H], B [N, r] fp16. need_l False: x only
    (l_q, l_v None)."""
    _need(a_q, "a_q", torch.float16)
    n, H = a_q.shape
    dev = a_q.device
    _need(a_v, "a_v", torch.float16, dev)
    for t, name in ((A_q, "A_q"), (B_q, "B_q"), (A_v, "A_v"), (B_v, "B_v")):
        _need(t, name, torch.float16, dev)
    r = A_q.shape[0]
    if a_v.shape != (n, H) or A_q.shape != (r, H) or A_v.shape != (r, H) \
            or B_q.shape[1] != r or B_v.shape[1] != r:
        raise ValueError("a [n, H], A [r, H] and B [N, r] for both adapters")
    Nq, Nv = B_q.shape[0], B_v.shape[0]
    x_q = torch.empty((n, r), device=dev, dtype=torch.float16)
    x_v = torch.empty((n, r), device=dev, dtype=torch.float16)
    l_q = torch.empty((n, Nq), device=dev, dtype=torch.float16) if need_l else None
    l_v = torch.empty((n, Nv), device=dev, dtype=torch.float16) if need_l else None
    if n:
        _lib.call("qlora_lora_fwd_rows", _ptr(a_q), _ptr(a_v), _ptr(A_q), _ptr(A_v), _ptr(B_q),
                  _ptr(B_v), _ptr(x_q), _ptr(x_v), _ptr(l_q), _ptr(l_v), n, Nq, Nv, H, r,
                  _stream(dev))
    return x_q, x_v, l_q, l_v


def _lora_bwd_rows(dqkv, q_cols, v_cols, at_q, bt_q, at_v, bt_v, scale, need_t=True):
    """(dx_q, dx_v, t_q, t_v) of the q and v adapters from the fused [dq|dk|dv] gradient:
    dx = fp16(fp16(g B) * s) [n, r], t = fp16(dx A) [n, H] (None without need_t); g = the
    adapter's columns (slices q_cols / v_cols of dqkv's columns). The adapter weights come
    transposed: at = A^T [H, r], bt = B^T [r, N] fp16 (contiguous)."""
    _need(dqkv, "dqkv", torch.float16, contiguous=False)
    n, C = dqkv.shape
    dev = dqkv.device
    if dqkv.stride(1) != 1:
        raise ValueError("dqkv must have unit column stride")
    for t, name in ((at_q, "at_q"), (bt_q, "bt_q"), (at_v, "at_v"), (bt_v, "bt_v")):
        _need(t, name, torch.float16, dev)
    H, r = at_q.shape
    Nq, Nv = q_cols.stop - q_cols.start, v_cols.stop - v_cols.start
    if at_v.shape != (H, r) or bt_q.shape != (r, Nq) or bt_v.shape != (r, Nv):
        raise ValueError("A^T must be [H, r] and B^T [r, N] for both adapters")
    if (2 * q_cols.start) % 16 or (2 * v_cols.start) % 16:
        raise ValueError("the adapters' columns must start on 16-byte boundaries")
    dx_q = torch.empty((n, r), device=dev, dtype=torch.float16)
    dx_v = torch.empty((n, r), device=dev, dtype=torch.float16)
    t_q = torch.empty((n, H), device=dev, dtype=torch.float16) if need_t else None
    t_v = torch.empty((n, H), device=dev, dtype=torch.float16) if need_t else None
    if n:
        base = dqkv.data_ptr()
        _lib.call("qlora_lora_bwd_rows", base + 2 * q_cols.start, base + 2 * v_cols.start,
                  dqkv.stride(0), _ptr(bt_q), _ptr(bt_v), _ptr(at_q), _ptr(at_v), _ptr(dx_q),
                  _ptr(dx_v), _ptr(t_q), _ptr(t_v), n, Nq, Nv, H, r, float(scale), _stream(dev))
    return dx_q, dx_v, t_q, t_v


def _lora_grad(dqkv, q_cols, v_cols, x_q, x_v, a_q, a_v, dx_q, dx_v, scale):
    """(dA_q, dB_q, dA_v, dB_v) fp32 of the q and v adapters: dB = s g^T x [N, r] and
    dA = dx^T a [r, H], g the adapter's columns of dqkv (engine.py:1327, 1329), in two launches
    for all four (fp32 sums of exact products, no fp16 rounding of the results)."""
    _need(dqkv, "dqkv", torch.float16, contiguous=False)
    n, C = dqkv.shape
    dev = dqkv.device
    if dqkv.stride(1) != 1:
        raise ValueError("dqkv must have unit column stride")
    for t, name in ((x_q, "x_q"), (x_v, "x_v"), (a_q, "a_q"), (a_v, "a_v"), (dx_q, "dx_q"),
                    (dx_v, "dx_v")):
        _need(t, name, torch.float16, dev)
    r = x_q.shape[1]
    H = a_q.shape[1]
    Nq, Nv = q_cols.stop - q_cols.start, v_cols.stop - v_cols.start
    for t, shape in ((x_q, (n, r)), (x_v, (n, r)), (dx_q, (n, r)), (dx_v, (n, r)),
                     (a_q, (n, H)), (a_v, (n, H))):
        if t.shape != shape:
            raise ValueError(f"expected {shape}, got {tuple(t.shape)}")
    f32 = torch.float32
    dB_q, dB_v = torch.empty((Nq, r), device=dev, dtype=f32), torch.empty((Nv, r), device=dev,
                                                                             dtype=f32)
    dA_q, dA_v = torch.empty((r, H), device=dev, dtype=f32), torch.empty((r, H), device=dev,
                                                                           dtype=f32)
    elems = ctypes.c_int64(0)
    _lib.call("qlora_lora_grad_workspace", n, Nq, Nv, H, r, ctypes.byref(elems))
    work = torch.empty((max(elems.value, 1),), device=dev, dtype=f32)
    base = dqkv.data_ptr()
    _lib.call("qlora_lora_grad", base + 2 * q_cols.start, base + 2 * v_cols.start,
              dqkv.stride(0), _ptr(x_q), _ptr(x_v), _ptr(a_q), _ptr(a_v), _ptr(dx_q), _ptr(dx_v),
              _ptr(dB_q), _ptr(dB_v), _ptr(dA_q), _ptr(dA_v), n, Nq, Nv, H, r, float(scale),
              _ptr(work), work.numel(), _stream(dev))
    return dA_q, dB_q, dA_v, dB_v


def _lora_grad_noalloc(dqkv, q_cols, v_cols, x_q, x_v, a_q, a_v, dx_q, dx_v, scale, out=None):
    """_lora_grad through qlora_lora_grad_noalloc: the partial sums in the library's static
    scratch instead of a workspace (no device allocation by the library; outputs allocated here
    unless `out` = (dA_q, dB_q, dA_v, dB_v) fp32 is given). Raises when the problem needs more
    scratch than the library holds."""
    _need(dqkv, "dqkv", torch.float16, contiguous=False)
    n, C = dqkv.shape
    dev = dqkv.device
    if dqkv.stride(1) != 1:
        raise ValueError("dqkv must have unit column stride")
    for t, name in ((x_q, "x_q"), (x_v, "x_v"), (a_q, "a_q"), (a_v, "a_v"), (dx_q, "dx_q"),
                    (dx_v, "dx_v")):
        _need(t, name, torch.float16, dev)
    r = x_q.shape[1]
    H = a_q.shape[1]
    Nq, Nv = q_cols.stop - q_cols.start, v_cols.stop - v_cols.start
    for t, shape in ((x_q, (n, r)), (x_v, (n, r)), (dx_q, (n, r)), (dx_v, (n, r)),
                     (a_q, (n, H)), (a_v, (n, H))):
        if t.shape != shape:
            raise ValueError(f"expected {shape}, got {tuple(t.shape)}")
    f32 = torch.float32
    if out is None:
        out = (torch.empty((r, H), device=dev, dtype=f32), torch.empty((Nq, r), device=dev, dtype=f32),
               torch.empty((r, H), device=dev, dtype=f32), torch.empty((Nv, r), device=dev, dtype=f32))
    dA_q, dB_q, dA_v, dB_v = out
    for t, shape, name in ((dA_q, (r, H), "dA_q"), (dB_q, (Nq, r), "dB_q"),
                           (dA_v, (r, H), "dA_v"), (dB_v, (Nv, r), "dB_v")):
        _need(t, name, f32, dev)
        if t.shape != shape:
            raise ValueError(f"{name} must be {shape}")
    base = dqkv.data_ptr()
    _lib.call("qlora_lora_grad_noalloc", base + 2 * q_cols.start, base + 2 * v_cols.start,
              dqkv.stride(0), _ptr(x_q), _ptr(x_v), _ptr(a_q), _ptr(a_v), _ptr(dx_q), _ptr(dx_v),
              _ptr(dB_q), _ptr(dB_v), _ptr(dA_q), _ptr(dA_v), n, Nq, Nv, H, r, float(scale),
              _stream(dev))
    return dA_q, dB_q, dA_v, dB_v


# ---------------------------------------------------------------------------------------------
# Varlen causal attention (engine.py:857-869)
# ---------------------------------------------------------------------------------------------
def _attn_shapes(q, k, v, packed):
    _need(q, "q", torch.float16)
    dev = q.device
    _need(k, "k", torch.float16, dev)
    _need(v, "v", torch.float16, dev)
    if q.dim() != 3 or k.dim() != 3 or k.shape != v.shape or k.shape[0] != q.shape[0] \
            or k.shape[2] != q.shape[2] or q.shape[1] % k.shape[1]:
        raise ValueError("q must be [n, HQ, D] and k, v [n, KH, D] with KH dividing HQ")
    cu = _need(packed.cu_seqlens, "packed.cu_seqlens", torch.int32, dev)
    if cu.dim() != 1 or cu.numel() < 1:
        raise ValueError("packed.cu_seqlens must be [sequences + 1]")
    return q.shape[0], q.shape[1], k.shape[1], q.shape[2], cu, dev


# Split of the attention's key ranges (qlora_attn_fwd_split / qlora_attn_bwd_split). Resident
# workgroups of the forward and dQ kernels: one per CU (their registers), 256 on an MI355X. A
# workgroup costs about two key blocks of fixed work (loads of its queries, the first block, the
# stores) plus one per block it walks (5.2 us for one 64-key block, +1.75 us per block, with few
# workgroups running). Measured on MI355X: with a sequence of 1024 (64 workgroups) chunks of 256
# keys take the forward from 35.7 to 25.8 us and dQ + dK/dV from 115 to 92 us, with one of 2048
# chunks of 512 keys 65.6 -> 53.3 and 212 -> 191 us; once the unsplit launch fills half the GPU
# (four sequences of up to 1024 tokens: 166 workgroups) every split was slower (each workgroup's
# key blocks take longer when more run at once, and the merge costs 8-12 us), so none is made.
ATTN_SLOTS = 256
ATTN_WG_BLOCKS = 2.0
ATTN_MAX_CHUNKS = 16
ATTN_MIN_CHUNK = 256


def attn_chunk(lengths, heads, block):
    """Keys per workgroup (a multiple of 64) for the split kernels, or 0 for no split: none when
    the unsplit launch already has half as many workgroups as the GPU holds, else the chunk of
    at least ATTN_MIN_CHUNK keys that minimises max(longest workgroup, total work / resident
    workgroups), over a batch of sequence `lengths`, `heads` (sequence, head) workgroup rows per
    tile, key blocks of `block` keys (64: forward, 32: dQ)."""
    lengths = [int(x) for x in lengths if x > 0]
    if not lengths:
        return 0
    max_len = max(lengths)
    nkb = []
    for L in lengths:  # tile t of 32 queries walks ceil(min(32 (t + 1), L) / block) blocks
        nkb += [-(-min(32 * (t + 1), L) // block) for t in range(-(-L // 32))]
    if len(nkb) * heads > ATTN_SLOTS // 2:
        return 0
    nkb = torch.tensor(nkb, dtype=torch.float64)
    best, best_cost = 0, None
    cands = [0] + [c for c in (256, 384, 512, 768, 1024, 1536, 2048, 3072, 4096, 6144, 8192)
                   if c >= ATTN_MIN_CHUNK and c < max_len and -(-max_len // c) <= ATTN_MAX_CHUNKS]
    for c in cands:
        per = c // block if c else int(nkb.max())
        nch = torch.ceil(nkb / per)
        total = float((nch * ATTN_WG_BLOCKS + nkb).sum()) * heads
        longest = ATTN_WG_BLOCKS + min(per, float(nkb.max())) + (0.3 * float(nch.max()) if c else 0)
        cost = max(longest, total / ATTN_SLOTS)
        if best_cost is None or cost < best_cost * 0.97:  # prefer fewer chunks on a near tie
            best, best_cost = c, cost
    return best


def _attn_plan(packed, kind, HQ, KH):
    """Chunk keys for `kind` ("fwd", "dq") of this batch, computed once per packed batch from the
    host-side lengths (0 when there are none)."""
    plans = getattr(packed, "_attn_plans", None)
    if plans is None:
        plans = {}
        try:
            packed._attn_plans = plans
        except AttributeError:
            pass
    key = (kind, HQ, KH)
    if key not in plans:
        cu = getattr(packed, "cu_seqlens_host", None)
        if cu is None:
            plans[key] = 0
        else:
            lengths = [b - a for a, b in zip(cu[:-1], cu[1:])]
            plans[key] = attn_chunk(lengths, KH, 64 if kind == "fwd" else 32)
    return plans[key]


def _attn_work(n, max_len, HQ, D, chunk, dev):
    """fp32 workspace of a split launch (partials of every chunk)."""
    we = ctypes.c_int64(0)
    _lib.call("qlora_attn_split_workspace", max_len, n, HQ, D, chunk, ctypes.byref(we))
    return torch.empty((max(we.value, 4),), device=dev, dtype=torch.float32)


def _attn_fwd(q, k, v, packed, scale):
    """(out [n, HQ, D] fp16, lse [HQ, n] fp32, None, None): causal attention within each
    sequence of cu_seqlens (engine.py:857-862; no dropout, so no Philox seed/offset). k and v
    may be in grouped layout [n, KH, D] (q head h reads kv head h // (HQ // KH)). With the
    lengths on the host, the key ranges of long tiles are split over several workgroups."""
    n, HQ, KH, D, cu, dev = _attn_shapes(q, k, v, packed)
    out = torch.empty_like(q)
    lse = torch.empty((HQ, n), device=dev, dtype=torch.float32)
    if n:
        nseq, max_len = cu.numel() - 1, int(packed.max_len)
        chunk = _attn_plan(packed, "fwd", HQ, KH)
        work = _attn_work(n, max_len, HQ, D, chunk, dev) if chunk else None
        _lib.call("qlora_attn_fwd_split", _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(lse),
                  _ptr(cu), nseq, max_len, n, HQ, KH, D, float(scale), chunk, _ptr(work),
                  work.numel() if work is not None else 0, _stream(dev))
    return out, lse, None, None


def _attn_bwd(dout, q, k, v, out, lse, seed, offset, packed, scale):
    """(dq, dk, dv) of _attn_fwd (engine.py:865-869); dk and dv are per q head [n, HQ, D], the
    gradient of the repeated k/v the reference's kernel sees (the RoPE backward sums each
    group)."""
    n, HQ, KH, D, cu, dev = _attn_shapes(q, k, v, packed)
    dout = dout.contiguous()
    _need(dout, "dout", torch.float16, dev)
    _need(out, "out", torch.float16, dev)
    _need(lse, "lse", torch.float32, dev)
    if dout.shape != q.shape or out.shape != q.shape or lse.shape != (HQ, n):
        raise ValueError("dout/out must match q and lse be [HQ, n]")
    dq = torch.empty_like(q)
    dk = torch.empty_like(q)
    dv = torch.empty_like(q)
    if n:
        nseq, max_len = cu.numel() - 1, int(packed.max_len)
        delta = torch.empty((HQ, n), device=dev, dtype=torch.float32)
        chunk = _attn_plan(packed, "dq", HQ, KH)
        work = _attn_work(n, max_len, HQ, D, chunk, dev) if chunk else None
        _lib.call("qlora_attn_bwd_split", _ptr(dout), _ptr(q), _ptr(k), _ptr(v), _ptr(out),
                  _ptr(lse), _ptr(delta), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(cu), nseq, max_len,
                  n, HQ, KH, D, float(scale), chunk, _ptr(work),
                  work.numel() if work is not None else 0, _stream(dev))
    return dq, dk, dv


def _rope_tables(packed, D, n, dev):
    cos, sin, pos = packed.cos, packed.sin, packed.pos
    _need(cos, "packed.cos", torch.float32, dev)
    _need(sin, "packed.sin", torch.float32, dev)
    _need(pos, "packed.pos", torch.int32, dev)
    if cos.dim() != 2 or cos.shape[1] != D // 2 or sin.shape != cos.shape or pos.numel() != n:
        raise ValueError("packed.cos/sin must be [positions, D/2] and packed.pos [n]")
    return cos, sin, pos


# ---------------------------------------------------------------------------------------------
# SwiGLU (engine.py:1012-1023)
# ---------------------------------------------------------------------------------------------
def _glu_fwd(gu, I, out=None):
    """m = silu(g) * u over the fused [g | u] (engine.py:1012-1017)."""
    _need(gu, "gu", torch.float16)
    n = gu.shape[0]
    if gu.shape != (n, 2 * I):
        raise ValueError("gu must be [n, 2I]")
    m = out if out is not None else torch.empty((n, I), device=gu.device, dtype=torch.float16)
    _need(m, "out", torch.float16, gu.device)
    if m.shape != (n, I):
        raise ValueError("out must be [n, I]")
    if n:
        _lib.call("qlora_glu_fwd", _ptr(gu), _ptr(m), n, I, _stream(gu.device))
    return m


def _glu_bwd(dm, gu, I):
    """In place: gu <- [dL/dg | dL/du] (engine.py:1020-1023)."""
    _need(gu, "gu", torch.float16)
    n = gu.shape[0]
    _need(dm, "dm", torch.float16, gu.device)
    if gu.shape != (n, 2 * I) or dm.shape != (n, I):
        raise ValueError("gu must be [n, 2I] and dm [n, I]")
    if n:
        _lib.call("qlora_glu_bwd", _ptr(dm), _ptr(gu), n, I, _stream(gu.device))


# ---------------------------------------------------------------------------------------------
# Cross-entropy head (engine.py:1026-1045)
# ---------------------------------------------------------------------------------------------
def _ce_outputs(rows, dev, tok_loss, entropy, correct, targets):
    _need(targets, "targets", torch.int64, dev)
    _need(tok_loss, "tok_loss", torch.float32, dev)
    _need(entropy, "entropy", torch.float32, dev)
    _need(correct, "correct", torch.int32, dev)
    for t, name in ((targets, "targets"), (tok_loss, "tok_loss"), (entropy, "entropy"),
                    (correct, "correct")):
        if t.numel() != rows:
            raise ValueError(f"{name} must have one entry per row")


def _ce(logits, targets, tok_loss, entropy, correct, zero_unsupervised=True):
    """Loss, entropy, accuracy of whole rows; logits overwritten with softmax - onehot
    (engine.py:1026-1030)."""
    _need(logits, "logits", torch.float16, contiguous=False)
    rows, V = logits.shape
    if rows == 0:
        return
    ld = _rows_view(logits, "logits", torch.float16, rows, V, logits.device)
    _ce_outputs(rows, logits.device, tok_loss, entropy, correct, targets)
    _lib.call("qlora_ce", _ptr(logits), ld, _ptr(targets), _ptr(tok_loss), _ptr(entropy),
              _ptr(correct), rows, V, int(zero_unsupervised), _stream(logits.device))


def _ce_piece(logits, w, targets, state, best_idx, xt, alpha, wt, v0, n_sup):
    """One vocabulary piece of the online cross-entropy (engine.py:1033-1038)."""
    _need(logits, "logits", torch.float16, contiguous=False)
    rows, width = logits.shape
    if rows == 0:
        return
    dev = logits.device
    ld = _rows_view(logits, "logits", torch.float16, rows, width, dev)
    _need(w, "w", torch.float16, dev)
    H = w.shape[1]
    if w.shape[0] != width:
        raise ValueError("w must be [width, H]")
    _need(targets, "targets", torch.int64, dev)
    _need(state, "state", torch.float32, dev)
    _need(best_idx, "best_idx", torch.int32, dev)
    _need(xt, "xt", torch.float32, dev)
    if state.shape != (rows, 4) or best_idx.numel() != rows or xt.numel() != rows \
            or targets.numel() != rows:
        raise ValueError("state must be [rows, 4]; best_idx, xt, targets [rows]")
    if n_sup:
        _need(alpha, "alpha", torch.float32, dev)
        _need(wt, "wt", torch.float16, dev)
        if alpha.numel() < n_sup or wt.shape[0] < n_sup or wt.shape[1] != H:
            raise ValueError("alpha must hold n_sup entries and wt [n_sup, H]")
    _lib.call("qlora_ce_piece", _ptr(logits), ld, _ptr(w), _ptr(targets), _ptr(state),
              _ptr(best_idx), _ptr(xt), _ptr(alpha), _ptr(wt), int(v0), rows, width,
              int(n_sup), H, _stream(dev))


def _ce_finish(state, best_idx, xt, targets, tok_loss, entropy, correct, acc, wt, dh, n_sup):
    """Loss, entropy, accuracy and dh = acc/s - W[target] after the last piece
    (engine.py:1041-1045)."""
    _need(state, "state", torch.float32)
    rows = state.shape[0]
    if rows == 0:
        return
    dev = state.device
    H = acc.shape[1]
    _ce_outputs(rows, dev, tok_loss, entropy, correct, targets)
    _need(best_idx, "best_idx", torch.int32, dev)
    _need(xt, "xt", torch.float32, dev)
    if n_sup:
        _need(acc, "acc", torch.float32, dev)
        _need(wt, "wt", torch.float16, dev)
        _need(dh, "dh", torch.float16, dev)
        if acc.shape[0] < n_sup or wt.shape != acc.shape or dh.shape[1] != H \
                or dh.shape[0] < n_sup:
            raise ValueError("acc, wt, dh must be [n_sup, H]")
    _lib.call("qlora_ce_finish", _ptr(state), _ptr(best_idx), _ptr(xt), _ptr(targets),
              _ptr(tok_loss), _ptr(entropy), _ptr(correct), _ptr(acc), _ptr(wt), _ptr(dh),
              rows, int(n_sup), H, _stream(dev))


def _ce_grad(logits, targets, state, v0, n_sup):
    """The gradient rows (< n_sup) of one recomputed vocabulary piece after _ce_finish, in place:
    fp16(e^(x - lse) - onehot) (for the embedding gradient; the reference freezes the
    embedding and has no such pass)."""
    _need(logits, "logits", torch.float16, contiguous=False)
    rows, width = logits.shape
    if n_sup == 0 or width == 0:
        return
    dev = logits.device
    ld = _rows_view(logits, "logits", torch.float16, rows, width, dev)
    _need(targets, "targets", torch.int64, dev)
    _need(state, "state", torch.float32, dev)
    if n_sup > rows or targets.numel() < n_sup or state.shape[0] < n_sup or state.shape[1] != 4:
        raise ValueError("targets and state must cover the n_sup rows")
    _lib.call("qlora_ce_grad", _ptr(logits), ld, _ptr(targets), _ptr(state), int(v0),
              int(n_sup), width, _stream(dev))
