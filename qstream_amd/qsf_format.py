"""QSF weight-payload writer: the byte formats the quantized matvec reads.

Restates the block quantizers of QStream's converter so that synthetic
weights have the exact on-disk layout engine.c hands to ``qsf_matvec_fn``:

* 2/4-bit asymmetric blocks ``[fp16 scale][fp16 min][packed codes]``
  (tools/convert_hf.py:215-262): scale = (max-min)/(2^b-1), codes =
  clip(round((w-min)/scale)) with numpy's half-to-even ``round``.
* 4-bit symmetric blocks ``[fp16 scale][2 B pad][nibbles]`` stored offset-8
  (tools/convert_hf.py:264-290).
* 3-bit blocks, LSB-first bitstream (tools/convert_hf.py:292-322).
* Outlier payloads ``[u32 n][n x (u32 flat_idx, u16 fp16)][blocks]``: the top
  ``frac`` of |w| are stored in fp16 and zeroed before block quantisation
  (tools/convert_hf.py:324-364).
* MXFP4 (quant type 11, added by this build): codes plane ``[rows][nblk][16]``
  with element 2j in the low nibble of byte j (tools/convert_hf.py:1456-1495),
  then an E8M0 scales plane ``[rows][nblk]``; quantised per OCP MX v1.0.

Blocks are laid out per row (``ceil(cols/bs)`` blocks each, last one partial),
which is what the kernels index (src/kernels_scalar.c:19-34).  For
``cols % bs == 0`` this equals the converter's flat blocking.
"""
from __future__ import annotations

import numpy as np

Q2, Q2SYM, Q3, Q4, Q4SYM = 0, 1, 2, 3, 4
Q2_OUTLIER, Q4_OUTLIER, MXFP4 = 9, 10, 11
QUANT_NAMES = {Q2: "2bit", Q3: "3bit", Q4: "4bit", Q4SYM: "4bit_sym",
               Q2_OUTLIER: "2bit_outlier", Q4_OUTLIER: "4bit_outlier", MXFP4: "mxfp4"}


def block_bytes(qt: int, bs: int) -> int:
    """src/quant.c:69-85 (the outlier types use their base type's block)."""
    if qt in (Q2, Q2SYM, Q2_OUTLIER):
        return 4 + (bs * 2 + 7) // 8
    if qt == Q3:
        return 4 + (bs * 3 + 7) // 8
    if qt in (Q4, Q4SYM, Q4_OUTLIER):
        return 4 + (bs * 4 + 7) // 8
    if qt == MXFP4:
        return 17
    raise ValueError(f"no fixed block for quant type {qt}")


def payload_bytes(qt: int, rows: int, cols: int, bs: int, n_outliers: int = 0) -> int:
    if qt == MXFP4:
        return rows * ((cols + 31) // 32) * 17
    nb = (cols + bs - 1) // bs
    dense = rows * nb * block_bytes(qt, bs)
    if qt in (Q2_OUTLIER, Q4_OUTLIER):
        return 4 + 6 * n_outliers + dense
    return dense


def _row_blocks(w: np.ndarray, bs: int) -> np.ndarray:
    """[rows, cols] -> [rows*nb, bs], zero-padding each row's last block."""
    rows, cols = w.shape
    nb = (cols + bs - 1) // bs
    pad = nb * bs - cols
    if pad:
        w = np.concatenate([w, np.zeros((rows, pad), np.float32)], axis=1)
    return np.ascontiguousarray(w, dtype=np.float32).reshape(rows * nb, bs)


def _fp16_bytes(v: np.ndarray) -> np.ndarray:
    return v.astype(np.float16).view(np.uint8).reshape(-1, 2)


def _asym_codes(blocks: np.ndarray, maxv: int):
    bmin = blocks.min(axis=1)
    bmax = blocks.max(axis=1)
    rng = bmax - bmin
    with np.errstate(divide="ignore", invalid="ignore"):
        scale = np.where(rng > 1e-30, rng / float(maxv), 0.0).astype(np.float32)
        inv = np.where(scale > 1e-30, 1.0 / scale, 0.0).astype(np.float32)
    vals = (blocks - bmin[:, None]) * inv[:, None]
    codes = np.clip(np.round(vals), 0, maxv).astype(np.uint8)
    return codes, scale, bmin


def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """Pack [nblk, bs] integer codes LSB-first (2/3/4-bit)."""
    nblk, bs = codes.shape
    c = codes.astype(np.uint32) & ((1 << bits) - 1)
    if bits == 4:
        return (c[:, 0::2] | (c[:, 1::2] << 4)).astype(np.uint8)
    if bits == 2:
        return (c[:, 0::4] | (c[:, 1::4] << 2) | (c[:, 2::4] << 4) | (c[:, 3::4] << 6)).astype(np.uint8)
    if bits == 3:
        # 8 codes -> 24 bits -> 3 bytes
        g = c.reshape(nblk, bs // 8, 8)
        word = np.zeros((nblk, bs // 8), np.uint32)
        for i in range(8):
            word |= g[:, :, i] << (3 * i)
        out = np.stack([(word >> (8 * j)) & 0xFF for j in range(3)], axis=-1)
        return out.reshape(nblk, bs * 3 // 8).astype(np.uint8)
    raise ValueError(bits)


def quantize_blocks(blocks: np.ndarray, qt: int) -> np.ndarray:
    """Quantise [nblk, bs] fp32 blocks to [nblk, block_bytes] uint8."""
    nblk, bs = blocks.shape
    if qt in (Q2, Q2SYM, Q4, Q3):
        bits = {Q2: 2, Q2SYM: 2, Q4: 4, Q3: 3}[qt]
        codes, scale, bmin = _asym_codes(blocks, (1 << bits) - 1)
        return np.concatenate([_fp16_bytes(scale), _fp16_bytes(bmin), pack_codes(codes, bits)], axis=1)
    if qt == Q4SYM:
        absmax = np.abs(blocks).max(axis=1)
        with np.errstate(divide="ignore", invalid="ignore"):
            scale = np.where(absmax > 1e-30, absmax / 7.0, 0.0).astype(np.float32)
            inv = np.where(scale > 1e-30, 1.0 / scale, 0.0).astype(np.float32)
        vals = np.clip(np.round(blocks * inv[:, None]), -7, 7).astype(np.int8)
        codes = (vals + 8).astype(np.uint8)  # offset-8 storage (convert_hf.py:276)
        pad = np.zeros((nblk, 2), np.uint8)
        return np.concatenate([_fp16_bytes(scale), pad, pack_codes(codes, 4)], axis=1)
    raise ValueError(f"quantize_blocks: unsupported quant type {qt}")


def quantize_matrix(w: np.ndarray, qt: int, bs: int, outlier_frac: float = 0.005) -> bytes:
    """Full tensor payload for ``qt`` as engine.c passes it to the matvec."""
    w = np.asarray(w, dtype=np.float32)
    if w.ndim == 1:
        w = w.reshape(1, -1)
    if qt == MXFP4:
        return quantize_mxfp4(w)
    if qt in (Q2_OUTLIER, Q4_OUTLIER):
        return quantize_outlier(w, qt, bs, outlier_frac)
    return quantize_blocks(_row_blocks(w, bs), qt).tobytes()


def quantize_outlier(w: np.ndarray, qt: int, bs: int, frac: float = 0.005,
                     indices: np.ndarray | None = None) -> bytes:
    """tools/convert_hf.py:324-364: n = max(1, int(N*frac)) largest |w| kept in
    fp16 (argpartition order), zeroed, remainder quantised at the base width."""
    rows, cols = w.shape
    flat = w.reshape(-1)
    n = max(1, int(flat.size * frac))
    if indices is None:
        indices = np.argpartition(np.abs(flat), -n)[-n:]
    indices = np.asarray(indices, dtype=np.int64)
    vals16 = flat[indices].astype(np.float16)
    clean = flat.copy()
    clean[indices] = 0.0
    table = np.zeros(len(indices), dtype=[("idx", "<u4"), ("val", "<u2")])
    table["idx"] = indices.astype(np.uint32)
    table["val"] = vals16.view(np.uint16)
    base = Q2 if qt == Q2_OUTLIER else Q4
    blocks = quantize_blocks(_row_blocks(clean.reshape(rows, cols), bs), base)
    return np.uint32(len(indices)).tobytes() + table.tobytes() + blocks.tobytes()


def outlier_payload(n_idx: np.ndarray, vals_f16_bits: np.ndarray, blocks: bytes) -> bytes:
    """Assemble an outlier payload from explicit entries (edge-case tests)."""
    table = np.zeros(len(n_idx), dtype=[("idx", "<u4"), ("val", "<u2")])
    table["idx"] = np.asarray(n_idx, dtype=np.uint32)
    table["val"] = np.asarray(vals_f16_bits, dtype=np.uint16)
    return np.uint32(len(n_idx)).tobytes() + table.tobytes() + bytes(blocks)


# ---- MXFP4 (OCP Microscaling Formats v1.0) --------------------------------
E2M1_MAG = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], np.float32)


# Rounding boundaries between consecutive E2M1 magnitudes; at a tie the
# even code wins, so the boundary above an even code is exclusive (>) and
# the one above an odd code inclusive (>=).
_E2M1_UP = ((0.25, False), (0.75, True), (1.25, False), (1.75, True),
            (2.5, False), (3.5, True), (5.0, False))


def _e2m1_encode(v: np.ndarray) -> np.ndarray:
    """Round fp32 to the nearest E2M1 value, ties to even code, saturating
    at 6 (codes: bit 3 sign, bits 2..0 the index into E2M1_MAG)."""
    mag = np.abs(v)
    code = np.zeros(v.shape, np.uint8)
    for edge, inclusive in _E2M1_UP:
        code += (mag >= edge) if inclusive else (mag > edge)
    sign = (np.signbit(v) & (code != 0)).astype(np.uint8) << 3
    return code | sign


def quantize_mxfp4(w: np.ndarray) -> bytes:
    """OCP MX: shared scale 2^(floor(log2(amax)) - 2) per 32 elements."""
    rows, cols = w.shape
    blocks = _row_blocks(w, 32)
    amax = np.abs(blocks).max(axis=1)
    with np.errstate(divide="ignore"):
        e = np.where(amax > 0, np.floor(np.log2(np.maximum(amax, 1e-38))) - 2, -127)
    e = np.clip(e, -127, 127).astype(np.int32)
    scaled = blocks / np.ldexp(np.float32(1.0), e)[:, None].astype(np.float32)
    codes = _e2m1_encode(scaled.astype(np.float32))
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    scales = (e + 127).astype(np.uint8)
    return packed.tobytes() + scales.tobytes()


def _mx_matrix(job) -> bytes:
    seed, e, i, rows, cols = job
    rng = np.random.default_rng([seed, e, i])
    return quantize_mxfp4(gaussian(rng, (rows, cols), 0.02))


def moe_experts(seed: int, n_exp: int, hidden: int, eid: int, workers: int | None = None):
    """Benchmark config 3's experts: per expert gate and up [eid][hidden] and
    down [hidden][eid], MXFP4-quantised N(0, 0.02) weights.  Each matrix has
    its own seed (seed, expert, matrix), so the result does not depend on
    how many worker processes (spawned, so safe beside an initialised GPU)
    build it."""
    import os
    jobs = [(seed, e, i, eid if i < 2 else hidden, hidden if i < 2 else eid)
            for e in range(n_exp) for i in range(3)]
    if workers is None:
        workers = min(16, os.cpu_count() or 1)
    if workers > 1 and len(jobs) > 4:
        import multiprocessing as mp
        with mp.get_context("spawn").Pool(min(workers, len(jobs))) as pool:
            mats = pool.map(_mx_matrix, jobs, chunksize=1)
    else:
        mats = [_mx_matrix(j) for j in jobs]
    return [{"gate": mats[3 * e], "up": mats[3 * e + 1], "down": mats[3 * e + 2]}
            for e in range(n_exp)]


def random_mxfp4(rng: np.random.Generator, rows: int, cols: int,
                 e_lo: int = 118, e_hi: int = 122) -> bytes:
    """Valid MXFP4 payload with uniform random codes and scales 2^(E-127),
    E in [e_lo, e_hi] (|w| ~ 0.02): same bytes per element as quantised
    N(0, 0.02) weights, generated without the fp32 intermediate."""
    nb = (cols + 31) // 32
    codes = rng.integers(0, 256, size=rows * nb * 16, dtype=np.uint8)
    scales = rng.integers(e_lo, e_hi + 1, size=rows * nb, dtype=np.uint8)
    return codes.tobytes() + scales.tobytes()


# ---- seeded synthetic inputs of the benchmark configs -----------------------
def gaussian(rng: np.random.Generator, shape, std: float = 1.0) -> np.ndarray:
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def heavy_tail_weights(rng: np.random.Generator, rows: int, cols: int,
                       frac: float = 0.005, std: float = 0.02, scale: float = 10.0) -> np.ndarray:
    """N(0, std) with a seeded ``frac`` of entries replaced by Student-t(3)
    samples scaled by ``scale*std`` (config 1's outlier injection)."""
    w = gaussian(rng, (rows, cols), std)
    n = int(rows * cols * frac)
    pos = rng.choice(rows * cols, size=n, replace=False)
    w.reshape(-1)[pos] = (rng.standard_t(3, size=n) * (scale * std)).astype(np.float32)
    return w


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded).astype(np.uint16)


# ---- the benchmark configs' seeded data --------
# bench.py times these and the GPU parity tests check the same bytes.
def config0_matrix(seed: int = 0):
    """Config 0: one 4-bit asymmetric 4096x4096 matrix, block 64, and x."""
    rng = np.random.default_rng(seed)
    w = gaussian(rng, (4096, 4096), 0.02)
    mats = [("w", np.frombuffer(quantize_matrix(w, Q4, 64), np.uint8), 4096, 4096)]
    return Q4, 64, mats, gaussian(rng, 4096)


def config1_matrices(seed: int = 1):
    """Config 1: the 2-bit+outlier gate and up projections, 11008x4096 each,
    block 64, with 0.5 % Student-t outliers, and x."""
    rng = np.random.default_rng(seed)
    mats = []
    for name in ("gate", "up"):
        w = heavy_tail_weights(rng, 11008, 4096)
        mats.append((name, np.frombuffer(quantize_matrix(w, Q2_OUTLIER, 64), np.uint8), 11008, 4096))
        del w
    return Q2_OUTLIER, 64, mats, gaussian(rng, 4096)


def config2_layer(seed: int = 2):
    """Config 2: one 7B decoder layer at 3-bit, block 128 -- q/k/v/o
    4096x4096, gate/up 11008x4096, down 4096x11008 (N(0, 0.02) weights)."""
    rng = np.random.default_rng(seed)
    shapes = [("q", 4096, 4096), ("k", 4096, 4096), ("v", 4096, 4096), ("o", 4096, 4096),
              ("gate", 11008, 4096), ("up", 11008, 4096), ("down", 4096, 11008)]
    mats = []
    for name, r, c in shapes:
        w = gaussian(rng, (r, c), 0.02)
        mats.append((name, np.frombuffer(quantize_matrix(w, Q3, 128), np.uint8), r, c))
        del w
    return Q3, 128, mats


# ---- QSF container (include/qsf/types.h:185-312) -----------------------------
# A test-data writer: the struct layouts the converter writes
# (tools/convert_hf.py:875-1258), packed little-endian, so the device
# loader can be checked on real files without a HuggingFace checkpoint.
QSF_MAGIC = 0x51534631
T_ATTN_Q, T_ATTN_K, T_ATTN_V, T_ATTN_O = 0, 1, 2, 3
T_FFN_GATE, T_FFN_UP, T_FFN_DOWN = 4, 5, 6
T_ATTN_NORM_W, T_FFN_NORM_W = 7, 9
T_MOE_ROUTER, T_MOE_ROUTER_BIAS = 21, 22
FP16 = 7
FFN_MOE = 3


def t_moe(e: int, role: str, bias: bool = False) -> int:
    """QSF_MOE_{GATE,UP,DOWN}[_BIAS](e) (include/qsf/types.h:145-162)."""
    return 23 + 6 * e + {"gate": 0, "up": 2, "down": 4}[role] + (1 if bias else 0)


def _crc32(b: bytes) -> int:
    import zlib
    return zlib.crc32(b) & 0xFFFFFFFF


def tensor_record(tensor_type: int, qt: int, rows: int, cols: int, payload: bytes) -> bytes:
    """[24-byte QSFTensorHeader][payload] (types.h:264-273)."""
    import struct
    return struct.pack("<HBBIIIII", tensor_type, qt, 0, rows, cols, len(payload), 0, 0) + bytes(payload)


def write_qsf(path: str, *, hidden: int, heads: int, vocab: int, inter: int, layers,
              quant_type: int, block_size: int = 64, kv_heads: int = 0, head_dim: int = 0,
              embedding=None, final_norm=None, output_head=None, tied: bool = False,
              activation: int = 2, norm_type: int = 2, pos_enc: int = 1, ffn_type: int = 1,
              rope_theta: float = 10000.0, eps: float = 1e-5, layer_crc: bool = True,
              header_crc: bool = True, compression=None, num_experts: int = 0,
              num_active_experts: int = 0, moe_norm_topk: int = 0, expert_dim: int = 0) -> dict:
    """Write a QSF file.  layers: per layer a list of (tensor_type, qt, rows,
    cols, payload); embedding: (qt, payload) of a [vocab][hidden] table;
    final_norm: fp16 array [hidden]; output_head: payload of a separate
    [vocab][hidden] head in quant_type.  Returns the section offsets."""
    import struct
    body = bytearray(b"\0" * 256)

    def align():
        while len(body) % 64:
            body.append(0)

    index = []
    for li, recs in enumerate(layers):
        align()
        off = len(body)
        data = b"".join(tensor_record(*r) for r in recs)
        body += data
        comp = (compression or {}).get(li, 0)
        crc = _crc32(data) if layer_crc else 0
        index.append(struct.pack("<QIIBBHIIfII8s", off, len(data), len(data), quant_type, comp,
                                 len(recs), crc, crc, 0.0, len(data), 0, b"\0" * 8))
    align()
    li_off = len(body)
    for e in index:
        body += e
    emb_off = 0
    if embedding is not None:
        align()
        emb_off = len(body)
        eqt, epay = embedding
        body += struct.pack("<IIIIBBBBIII", eqt, 0, vocab, hidden, 0, 0, 0, 0, _crc32(bytes(epay)), 1,
                            vocab)
        body += bytes(epay)
    fin_off = 0
    if final_norm is not None:
        align()
        fin_off = len(body)
        norm = np.ascontiguousarray(final_norm, np.float16).tobytes()
        head = b"" if (tied or output_head is None) else bytes(output_head)
        body += struct.pack("<IIII", 1 if tied else 0, len(norm), len(head), _crc32(norm + head))
        body += norm + head
    h = bytearray(256)
    struct.pack_into("<IIIIIIIIIIII", h, 0, QSF_MAGIC, 1, 256, 1, len(layers), hidden, heads,
                     kv_heads, vocab, 4096, inter, head_dim)
    struct.pack_into("<BBBBffI", h, 48, quant_type, activation, norm_type, pos_enc, rope_theta, eps,
                     block_size)
    struct.pack_into("<QQQQQQQ", h, 64, li_off, emb_off, fin_off, 0, 0, 0, 0)
    struct.pack_into("<BBBB", h, 140, 0, ffn_type, 0, 1 if tied else 0)
    struct.pack_into("<I", h, 156, 1 if tied else 0)
    struct.pack_into("<Q", h, 160, len(body))
    h[172] = 1
    struct.pack_into("<BBBBI", h, 173, num_experts, num_active_experts, moe_norm_topk, 0, expert_dim)
    struct.pack_into("<I", h, 168, _crc32(bytes(h[:168])) if header_crc else 0)
    body[:256] = h
    with open(path, "wb") as f:
        f.write(body)
    return {"layer_index": li_off, "embedding": emb_off, "final": fin_off, "size": len(body),
            "layer_offsets": [struct.unpack_from("<Q", e)[0] for e in index]}

