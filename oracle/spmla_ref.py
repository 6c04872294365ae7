"""CPU oracle for the dotsnote FP8 sparse-MLA path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as the checker
(or as the timed CPU baseline); the product path (arcagi2_flashnext_dots3_amd) never calls it.

Every function restates the reference algorithm (numpy, float64 accumulation unless stated) and cites the reference
file:line it follows (paths relative to the reference repository root). How each function is pinned independently
of its own formula (library routines, invariants, brute force) is listed in `PINS` and exercised by
tests/test_oracle.py.
"""
import numpy as np

D_LAT, D_ROPE, D_QK = 512, 64, 576
ROW656, ROW576, ROW400, KEYROW = 656, 576, 400, 132
SC_OFF, ROPE_OFF = 512, 528
R4_SIGN, R4_K, R4_ROPE = 256, 320, 336
LOG2E = 1.4426950408889634
LN2 = 0.6931471805599453

PINS = {
    "e4m3_encode": "torch.Tensor.to(float8_e4m3fn) over every fp32 with |x| in [2^-12, 512) and signed specials",
    "e4m3_decode": "torch float8_e4m3fn -> float32 on all 256 codes",
    "e4m3_to_bf16_bits": "torch float8_e4m3fn -> bfloat16 on all 256 codes",
    "bf16": "torch bfloat16 conversions",
    "f32_to_bf16_bits": "torch float32 -> bfloat16 on 65K random fp32 over the full exponent range, 4096 exact ties "
                        "and the specials (NaN stays NaN); tests/test_oracle_helpers.py",
    "bf16_bits_to_f32": "torch bfloat16 -> float32 on the same values; tests/test_oracle_helpers.py",
    "okey": "sorting by the key orders finite fp32 as numpy does, -0 below +0, NaN largest; "
            "tests/test_oracle_helpers.py",
    "dequant_656": "torch float8_e4m3fn decode times the row's fp32 scales, rope via torch bfloat16; "
                   "tests/test_oracle_helpers.py",
    "dequant_576": "torch float8_e4m3fn decode of all 576 bytes; tests/test_oracle_helpers.py",
    "row400_unpack": "unpack(pack(x)) == x and the element-by-element byte layout (row400_pack's checks); "
                     "tests/test_oracle_row400.py",
    "row400_dequant": "the 16-value e2m2 grid x 2^k by hand; every value exact in e4m3 / bf16; "
                      "tests/test_oracle_row400.py",
    "bmm_fp8_weights": "torch (float8 -> float32) * scale -> bfloat16 on random codes and scales; "
                       "tests/test_oracle_mla.py",
    "shuffle_rows": "shuffle_rows(shuffle_layout(rows)) == rows; tests/test_oracle_shuffle.py",
    "index_key_write_shuffle": "equals index_key_write into 132-byte rows followed by shuffle_layout; "
                               "tests/test_oracle_shuffle.py",
    "paged_ctx": "hand values of (request, visible keys) per token for decode and MTP (next_n) batches; "
                 "tests/test_oracle_shuffle.py",
    "cache_write_656": "dequantized row within half an e4m3 ulp of x / s; per-group max code == 448 (0x7e); "
                       "zero groups; rope bit copy; slot skipping",
    "cache_write_576": "e4m3 of the clamped value (library encoder) ; rope codes",
    "index_key_write": "same closed-form checks as cache_write_656 with s = max(amax, 1e-4) / 448; UE8M0 power of 2",
    "row400_quant": "float64 brute force: k = smallest integer with fp32(amax / 7) <= 2^k (IEEE division from numpy), "
                    "magnitude = nearest point of the 16-value e2m2 grid x 2^k with ties to the larger (and the one "
                    "fp32 rounding of z + 0.5 the reference's arithmetic makes, shown by hand examples)",
    "row400_pack": "the byte layout written out element by element (nibble / bit / exponent / rope positions); "
                   "unpack(pack(x)) == x",
    "row400_to_e4m3": "the dequantized value has at most 3 mantissa bits: e4m3 decode of the code equals it exactly "
                      "in e4m3's normal range; round trip |dequant(quant(x)) - x| <= half a grid step",
    "cache_write_400": "row400_quant + row400_pack of the scaled, clamped input; rope as cache_write_576",
    "row400_gather": "decode of every row equals the Row576 row a direct Row576 write of the dequantized values gives",
    "bmm_fp8": "torch statement of the reference's dequantization ((float8 -> float32) * scale -> bfloat16, all "
               "library conversions) and torch.matmul in float64; a python triple loop on a tiny case",
    "wcache_step2": "reduces to wcache_step when the second sets are the first ones' (identical hits / misses); a "
                    "hand-worked W = 1 example; tests/test_oracle_wcache.py",
    "wcache_verify2": "a sequential simulation of the two-choice ticket rule under random miss orders always passes; "
                      "planted mistakes (no second-set ticket, a pinned line replaced, a row placed in a third set, "
                      "a wrong rr advance, a miscounted spill) each fail; tests/test_oracle_wcache.py",
    "wcache_set2": "hand values of ((h * 2654435761) >> 12) % S, including rows near 2^31 (64-bit product); "
                   "tests/test_oracle_wcache.py",
    "wcache_step": "hand-worked W = 2 examples (hit, pin, round-robin replacement, overflow to spill); a sequential "
                   "simulation of ticketed placement under random miss orders reproduces every order-independent output",
    "attention": "torch.nn.functional.scaled_dot_product_attention (float64) on dequantized rows + torch.logsumexp;"
                 " brute-force python loops on tiny cases; invariance under permutation of the selected rows",
    "lse_merge": "merge of disjoint splits == single-pass attention (exact math), single part == identity",
    "index_logits": "python triple loop on tiny cases; linearity in w; block-table indirection vs a flat store",
    "topk": "torch.topk value sets; python sorted() with the (value desc, index asc) key on tiny / tie-heavy rows; "
            "fp16 logits: widened exactly to fp32, whose order equals the fp16 order (python float comparison over "
            "all 65536 fp16 patterns, NaN largest, -0 < +0)",
    "topk_local": "brute force python sort on tiny rows; at P = 1 the local + merge pair equals topk",
    "topk_merge": "python sorted() over concatenated candidates; merge(local(x)) == topk(x) at P = 1",
    "rows_from_topk": "python loop over the block table",
    "compact_stage": "torch.unique(sorted=True, return_inverse=True) (library)",
    "gather": "numpy fancy indexing",
    "tier_split": "python loop with stable order",
    "shuffle_layout": "the reference reader's byte offsets (16-token x 16-byte tiles, scales after the codes) written "
                      "out element by element; shuffle_rows(shuffle_layout(x)) == x",
    "paged_mqa_logits": "index_logits (pinned above) on the unshuffled rows with the reader's context rule "
                        "(seq_len - (next_n - 1 - j), or the 2-D seq_lens entry) checked by hand; no clamp",
    "mqa_logits": "index_logits (pinned above) on 132-byte rows built from the flat codes and scales, block size 1 and "
                  "an identity block table, with positions below ks masked",
    "mtp_union": "python sets on tiny requests (every selected valid row exactly once, its mask = the tokens whose "
                 "list holds it); the order checked by its definition (mask descending, then first position)",
    "topk_overlap": "the reference's own statement (sort, searchsorted, gather-compare, torch) on random rows with "
                    "-1 padding; python set arithmetic on tiny rows; symmetry, hits <= min(|a|, |b|), identical rows "
                    "give |a|, disjoint rows give 0",
}


# ------------------------------------------------------------------------------------------------ scalars
def bf16_bits_to_f32(b):
    """uint16 bf16 bit patterns -> float32 (exact)."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x):
    """float32 -> bf16 bits, round to nearest even (NaN kept quiet)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def e4m3_encode(x):
    """float32 -> OCP e4m3fn codes, round to nearest even; |x| rounding past 448 and inf/NaN -> 0x7f | sign.
    Integer restatement of the format (bias 7, 3 mantissa bits, subnormals m * 2^-9). The reference converts with
    torch's / Triton's RNE float8e4nv casts: sparse_offload.py:263-266, shard_indexer.py:59,
    dotsnote/training/finetune/student.py:87."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.int64)
    sign = (u >> 24) & 0x80
    a = u & 0x7FFFFFFF
    e = (a >> 23) - 127
    out = np.zeros(a.shape, dtype=np.int64)
    # normal range
    q = a >> 20
    r = a & 0xFFFFF
    q = q + ((r > 0x80000) | ((r == 0x80000) & ((q & 1) == 1))).astype(np.int64)
    code_n = q - ((127 - 7) << 3)
    code_n = np.where(code_n > 0x7E, 0x7F, code_n)
    # subnormal range: value * 2^9 rounded to an integer 0..8
    M = (a & 0x7FFFFF) | 0x800000
    s = np.clip(14 - e, 0, 63)
    s_ok = (e < -6) & (e >= -126) & (s <= 25)
    sm = np.where(s_ok, s, 25)
    qs = M >> sm
    rs = M & ((np.int64(1) << sm) - 1)
    half = np.int64(1) << (sm - 1)
    qs = qs + ((rs > half) | ((rs == half) & ((qs & 1) == 1))).astype(np.int64)
    code_s = np.where(s_ok, qs, 0)
    out = np.where(e >= -6, code_n, code_s)
    out = np.where(a >= 0x7F800000, 0x7F, out)
    return (out | sign).astype(np.uint8)


_E4M3_TABLE = None


def e4m3_to_bf16_bits(c):
    """e4m3fn codes -> bf16 bit patterns (exact: e4m3 values have at most 4 significant bits); the NaN codes 0x7f /
    0xff -> the canonical bf16 NaN 0x7fc0 (torch's float8_e4m3fn -> bfloat16 conversion)."""
    c = np.asarray(c, dtype=np.uint8)
    b = (e4m3_decode(c).view(np.uint32) >> 16).astype(np.uint16)
    return np.where((c & 0x7F) == 0x7F, np.uint16(0x7FC0), b).astype(np.uint16)


def e4m3_decode(c):
    """e4m3fn codes -> float32 (exact): (-1)^s 2^(e-7)(1 + m/8), subnormal m 2^-9, 0x7f/0xff NaN."""
    global _E4M3_TABLE
    if _E4M3_TABLE is None:
        t = np.zeros(256, dtype=np.float32)
        for code in range(256):
            s = -1.0 if code & 0x80 else 1.0
            e, m = (code >> 3) & 15, code & 7
            if e == 15 and m == 7:
                t[code] = np.nan
            elif e == 0:
                t[code] = s * m * 2.0 ** -9
            else:
                t[code] = s * 2.0 ** (e - 7) * (1 + m / 8)
        _E4M3_TABLE = t
    return _E4M3_TABLE[np.asarray(c, dtype=np.uint8)]


# ------------------------------------------------------------------------------------------------ KV write
def _row_index(slot, block_size, R):
    return slot


def cache_write_656(kv_bits, pe_bits, slots, cache):
    """Row656 quantize-and-pack into cache [R, 656] uint8 (in place); slots < 0 or >= R skipped.
    Per 128 latent values: s = max(amax / 448, 1e-12) in fp32 (dotsnote/training/finetune/student.py:85-87:
    clamp_min(amax / 448, 1e-12), (x / s).to(float8_e4m3fn)); layout [512 codes | 4 fp32 s | 64 bf16 rope]
    (dotsnote/engine/vllm_patch/vllm/v1/hisparse/runtime.py:35-36)."""
    R = cache.shape[0]
    x = bf16_bits_to_f32(kv_bits).reshape(-1, 4, 128)
    amax = np.abs(x).max(-1)
    s = np.maximum((amax / np.float32(448.0)).astype(np.float32), np.float32(1e-12)).astype(np.float32)
    codes = e4m3_encode((x / s[..., None]).astype(np.float32)).reshape(-1, 512)
    for i, slot in enumerate(np.asarray(slots).tolist()[: x.shape[0]]):
        if slot < 0 or slot >= R:
            continue
        row = cache[slot]
        row[:512] = codes[i]
        row[512:528] = s[i].astype(np.float32).view(np.uint8)
        row[528:656] = np.asarray(pe_bits[i], dtype=np.uint16).view(np.uint8)
    return cache


def cache_write_576(kv_bits, pe_bits, slots, cache, kv_scale=1.0):
    """Row576 (the reference's deployed row, dotsnote/engine/arcstats_pkg/arcstats/sparse_offload.py:252-270):
    e4m3_rne(clamp(x * (1 / kv_scale), -448, 448)) for latent and rope."""
    R = cache.shape[0]
    inv = np.float32(1.0 / kv_scale)
    x = bf16_bits_to_f32(kv_bits) * inv
    y = bf16_bits_to_f32(pe_bits).reshape(x.shape[0], -1) * inv
    cx = e4m3_encode(np.clip(x, -448, 448).astype(np.float32))
    cy = e4m3_encode(np.clip(y, -448, 448).astype(np.float32))
    for i, slot in enumerate(np.asarray(slots).tolist()[: x.shape[0]]):
        if 0 <= slot < R:
            cache[slot, :512] = cx[i]
            cache[slot, 512:576] = cy[i]
    return cache


def index_key_write(k_bits, slots, store, P=1, rank=0, ue8m0=False):
    """Indexer key rows [128 codes | fp32 s], s = max(amax, 1e-4) / 448 (UE8M0: 2^ceil(log2 s)), owner slot % P,
    local row slot // P (dotsnote/engine/arcstats_pkg/arcstats/shard_indexer.py:42-60)."""
    x = bf16_bits_to_f32(k_bits).reshape(-1, 128)
    s = (np.maximum(np.abs(x).max(-1), np.float32(1e-4)) / np.float32(448.0)).astype(np.float32)
    if ue8m0:
        u = s.view(np.uint32).astype(np.int64)
        up = (u & 0x7FFFFF) != 0
        u = np.where(up, (u & 0xFF800000) + 0x800000, u)
        s = u.astype(np.uint32).view(np.float32)
    codes = e4m3_encode((x / s[:, None]).astype(np.float32))
    Rl = store.shape[0]
    for i, slot in enumerate(np.asarray(slots).tolist()[: x.shape[0]]):
        if slot < 0 or slot % P != rank or slot // P >= Rl:
            continue
        r = slot // P
        store[r, :128] = codes[i]
        store[r, 128:132] = s[i:i + 1].view(np.uint8)
    return store


# ------------------------------------------------------------------------------------------------ Row400 codec
def row400_quant(x):
    """x float32 [N, 512] (already scaled by 1 / kv_scale and clamped to +-448) -> (codes int64 [N, 512]: sign << 4 |
    magnitude index, k int64 [N, 16]: block exponents). The reference's compact-row quantizer with M = 2, BLK = 32
    (dotsnote/engine/arcstats_pkg/arcstats/offload_rowfmt.py:81-104 _quant, torch statement ref_quant :336-360),
    in fp32 arithmetic: k is the smallest integer with 2^k >= fp32(amax / 7) (zero / subnormal quotients: -126),
    y = |x| 2^-k; y < 1: floor(4y + 0.5); else e2 = [y >= 2] + [y >= 4], ((e2 + 1) << 2) + floor(y / 2^(e2-2) + 0.5)
    - 4; capped at 15; the sign bit only for x < 0 with a nonzero magnitude."""
    x = np.asarray(x, dtype=np.float32)
    N = x.shape[0]
    ax = np.abs(x).reshape(N, 16, 32)
    r = (ax.max(-1) / np.float32(7.0)).astype(np.float32)
    rb = r.view(np.uint32).astype(np.int64)
    e = ((rb >> 23) & 255) - 127
    k = e + ((rb & 0x7FFFFF) != 0).astype(np.int64)
    k = np.where(e < -126, -126, np.minimum(k, 127))
    inv = ((127 - k).astype(np.uint32) << 23).view(np.float32)           # 2^-k
    y = (ax * inv[..., None]).astype(np.float32).reshape(N, 512)
    sub = np.floor((y * np.float32(4.0) + np.float32(0.5)).astype(np.float32)).astype(np.int64)
    e2 = (y >= 2).astype(np.int64) + (y >= 4).astype(np.int64)
    inv_stp = ((127 + 2 - e2).astype(np.uint32) << 23).view(np.float32)  # 2^(2 - e2)
    mant = np.floor((y * inv_stp + np.float32(0.5)).astype(np.float32)).astype(np.int64)
    nrm = ((e2 + 1) << 2) + mant - 4
    mag = np.minimum(np.where(y < 1, sub, nrm), 15)
    code = np.where((x < 0) & (mag > 0), mag | 16, mag)
    return code.astype(np.int64), k.astype(np.int64)


def row400_pack(code, k, rope_codes):
    """codes [N, 512], k [N, 16], rope e4m3 codes [N, 64] -> Row400 bytes [N, 400] (offload_rowfmt.py:118-128 and
    ref_pack :366-388 with M = 2): byte e/2 holds the magnitude nibble of value e (low nibble for even e), byte
    256 + e/8 bit e%8 its sign, bytes 320 + b the int8 exponents, 336.. the rope codes."""
    code = np.asarray(code, dtype=np.int64)
    N = code.shape[0]
    out = np.zeros((N, ROW400), dtype=np.uint8)
    lo = (code & 15).reshape(N, 256, 2)
    out[:, :256] = (lo[..., 0] | (lo[..., 1] << 4)).astype(np.uint8)
    sg = ((code >> 4) & 1).reshape(N, 64, 8)
    out[:, R4_SIGN:R4_K] = sum(sg[..., j] << j for j in range(8)).astype(np.uint8)
    out[:, R4_K:R4_ROPE] = np.asarray(k, dtype=np.int64).astype(np.int8).view(np.uint8)
    out[:, R4_ROPE:] = np.asarray(rope_codes, dtype=np.uint8)
    return out


def row400_unpack(rows):
    """Row400 bytes [N, 400] -> (codes [N, 512], k [N, 16], rope codes [N, 64])."""
    rows = np.asarray(rows, dtype=np.uint8)
    N = rows.shape[0]
    b = rows[:, :256].astype(np.int64)
    lo = np.stack([b & 15, b >> 4], -1).reshape(N, 512)
    sb = rows[:, R4_SIGN:R4_K].astype(np.int64)
    sg = np.stack([(sb >> j) & 1 for j in range(8)], -1).reshape(N, 512)
    k = rows[:, R4_K:R4_ROPE].copy().view(np.int8).astype(np.int64)
    return lo | (sg << 4), k, rows[:, R4_ROPE:].copy()


def row400_dequant(code, k):
    """codes / block exponents -> float32 values before the e4m3 cast (offload_rowfmt.py:149-157, ref_dequant
    :363-372): mant = (e2 ? 4 + m : m), value = mant * 2^clamp(max(e2, 1) - 3 + k, -126, 127), signed, clamped to
    +-448 (fp32: an exponent of 127 with mant >= 2 overflows to inf and clamps to 448)."""
    code = np.asarray(code, dtype=np.int64)
    mag = code & 15
    e2, mm = mag >> 2, mag & 3
    mant = np.where(e2 > 0, mm + 4, mm)
    ex = np.clip(np.maximum(e2, 1) - 3 + np.repeat(np.asarray(k, dtype=np.int64), 32, axis=1), -126, 127)
    with np.errstate(over="ignore"):
        v = np.ldexp(mant.astype(np.float32), ex.astype(np.int32)).astype(np.float32)
    v = np.where(((code >> 4) & 1) != 0, -v, v)
    return np.clip(v, -448, 448).astype(np.float32)


def row400_to_e4m3(code, k):
    """The GPU (Row576) latent codes of compact values: e4m3 RNE of row400_dequant (offload_rowfmt.py:158)."""
    return e4m3_encode(row400_dequant(code, k))


def cache_write_400(kv_bits, pe_bits, slots, cache, kv_scale=1.0):
    """Row400 quantize-and-pack (offload_rowfmt.py:107-129 _store_kernel): x = clamp(v * inv_scale, +-448) (fp32,
    inv_scale = 1 / kv_scale in fp32), latent by row400_quant, rope e4m3_rne of the same clamp as Row576."""
    R = cache.shape[0]
    inv = np.float32(1.0) / np.float32(kv_scale)
    x = np.clip((bf16_bits_to_f32(kv_bits) * inv).astype(np.float32), -448, 448).astype(np.float32)
    y = np.clip((bf16_bits_to_f32(pe_bits).reshape(x.shape[0], -1) * inv).astype(np.float32), -448, 448)
    code, k = row400_quant(x)
    rows = row400_pack(code, k, e4m3_encode(y.astype(np.float32)))
    for i, slot in enumerate(np.asarray(slots).tolist()[: x.shape[0]]):
        if 0 <= slot < R:
            cache[slot] = rows[i]
    return cache


def row400_gather(src, rows, fmt=576):
    """GPU rows of compact rows src[rows[i]] (zero row outside [0, R)): fmt 576 = the reference's Row576 GPU row
    (offload_rowfmt.py:163-185 _put_rows / _rows_kernel MODE 0), fmt 656 = the same values as Row656 (e4m3 codes,
    scales 1.0, rope widened to bf16)."""
    src = np.asarray(src, dtype=np.uint8)
    rows = np.asarray(rows, dtype=np.int64)
    ok = (rows >= 0) & (rows < src.shape[0])
    code, k, rope = row400_unpack(src[np.where(ok, rows, 0)])
    lat = row400_to_e4m3(code, k)
    if fmt == 576:
        out = np.concatenate([lat, rope], 1).astype(np.uint8)
    else:
        sc = np.ones((rows.shape[0], 4), dtype=np.float32).view(np.uint8)
        rb = e4m3_to_bf16_bits(rope).view(np.uint8)
        out = np.concatenate([lat, sc, rb], 1).astype(np.uint8)
    out[~ok] = 0
    return out


# ------------------------------------------------------------------------------------------------ dequant
def dequant_656(rows):
    """Row656 bytes [n, 656] -> (latent [n, 512] float64, rope [n, 64] float64)."""
    rows = np.asarray(rows, dtype=np.uint8)
    codes = e4m3_decode(rows[:, :512]).astype(np.float64).reshape(-1, 4, 128)
    sc = rows[:, 512:528].copy().view(np.float32).astype(np.float64)
    lat = (codes * sc[:, :, None]).reshape(-1, 512)
    rope = bf16_bits_to_f32(rows[:, 528:656].copy().view(np.uint16)).astype(np.float64)
    return lat, rope


def dequant_576(rows, kv_scale=1.0):
    rows = np.asarray(rows, dtype=np.uint8)
    v = e4m3_decode(rows[:, :576]).astype(np.float64)
    return v[:, :512], v[:, 512:]


# ------------------------------------------------------------------------------------------------ attention
def attention(q, pool, idx, sm_scale, kv_scale=1.0, kcount=None, fmt=656):
    """Sparse MLA over gathered rows (dotsnote/kaggle/runtime_dataset/bench_offload_attn2.py:77-93: gather rows,
    s = q . row * scale, masked softmax in base 2, o = p V / sum p, x kv_scale; LSE of the same scores as in
    dotsnote/engine/vllm_patch/vllm/v1/attention/ops/xpu_mla_sparse.py:155-161). float64.
    q [T, H, 576] float (values of the bf16 query), pool [R, 656|576] uint8, idx [T, K] (valid iff 0 <= idx < R;
    with kcount only the first kcount[t] entries). Returns out [T, H, 512], lse [T, H] (natural log).
    No valid entry: out = 0, lse = -inf (the reference's split kernel gives o = 0, csrc/offload_attn.cu:446)."""
    q = np.asarray(q, dtype=np.float64)
    T, H, _ = q.shape
    R = pool.shape[0]
    idx = np.asarray(idx)
    K = idx.shape[1]
    out = np.zeros((T, H, 512))
    lse = np.full((T, H), -np.inf)
    for t in range(T):
        kk = K if kcount is None else min(K, int(kcount[t]))
        sel = idx[t, :kk].astype(np.int64)
        v = sel[(sel >= 0) & (sel < R)]
        if v.size == 0:
            continue
        if fmt == 656:
            lat, rope = dequant_656(pool[v])
        else:
            lat, rope = dequant_576(pool[v])
        rows = np.concatenate([lat, rope], 1)
        s = (q[t] @ rows.T) * (sm_scale * kv_scale)          # [H, n]
        m = s.max(1, keepdims=True)
        p = np.exp(s - m)
        l = p.sum(1, keepdims=True)
        out[t] = (p @ lat) / l * kv_scale
        lse[t] = (m + np.log(l))[:, 0]
    return out, lse


def lse_merge(parts, lses):
    """o = sum_i exp(lse_i - L) o_i, L = log sum_i exp(lse_i); all -inf -> o = 0, L = -inf
    (dotsnote/engine/arcstats_pkg/arcstats/sparse_offload.py:519-538 in natural-log form)."""
    parts = np.asarray(parts, dtype=np.float64)
    lses = np.asarray(lses, dtype=np.float64)
    M = lses.max(0)
    finite = np.isfinite(M)
    Ms = np.where(finite, M, 0.0)
    w = np.where(np.isfinite(lses), np.exp(lses - Ms[None]), 0.0)
    L = w.sum(0)
    o = (w[..., None] * np.nan_to_num(parts)).sum(0) / np.where(L > 0, L, 1.0)[..., None]
    o = np.where((L > 0)[..., None], o, 0.0)
    lse = np.where(L > 0, Ms + np.log(np.where(L > 0, L, 1.0)), -np.inf)
    return o, lse


# ------------------------------------------------------------------------------------------------ indexer
def index_logits(q, w, store, block_table, block_size, req, ctx, Lc, P=1, rank=0, clamp=60000.0):
    """logit[row, j] = min(sum_h w[row, h] * relu(q[row, h] . kcode) * kscale, 60000) for pos = j * P + rank <
    ctx[row], -inf otherwise (dotsnote/engine/arcstats_pkg/arcstats/shard_logits_v2.py:84-100,
    shard_indexer.py:77-91; torch statement dotsnote/training/finetune/student.py:220-221). float64.
    store [R_local, 132] uint8; key of pos: block = block_table[req, pos // bs], local row (block*bs + pos%bs) // P."""
    q = np.asarray(q, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    rows = q.shape[0]
    out = np.full((rows, Lc), -np.inf)
    Rl = store.shape[0]
    for r in range(rows):
        j = np.arange(Lc)
        pos = j * P + rank
        ok = pos < ctx[r]
        j, pos = j[ok], pos[ok]
        if j.size == 0:
            continue
        blk = np.asarray(block_table)[req[r], pos // block_size].astype(np.int64)
        lrow = (blk * block_size + pos % block_size) // P
        ok2 = (blk >= 0) & (lrow < Rl)
        j, lrow = j[ok2], lrow[ok2]
        kc = e4m3_decode(store[lrow, :128]).astype(np.float64)
        ks = store[lrow, 128:132].copy().view(np.float32)[:, 0].astype(np.float64)
        s = np.maximum(q[r] @ kc.T, 0.0)                       # [H, n]
        lg = (w[r] @ s) * ks
        out[r, j] = np.minimum(lg, clamp)
    return out


def okey(x):
    """torch's order-preserving uint32 key of fp32 (-0 < +0, NaN largest): csrc/topk_select.cu:21-30 semantics."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    k = np.where(u & 0x80000000, (~u) & 0xFFFFFFFF, u | 0x80000000)
    return np.where(np.isnan(np.asarray(x, dtype=np.float32)), 0xFFFFFFFF, k).astype(np.uint64)


def topk(logits, ctx, K):
    """Per row: the K largest of columns j < min(ctx, Lc) (key okey, equal keys -> lower column), output sorted by
    (value desc, column asc), -1 for +-inf values and for missing slots (fast_topk.py:10-14 tie rule; merge
    semantics csrc/topk_select.cu:13-15, :305-321; shard_indexer.py:212-221 maps +-inf to -1). fp16 logits (the
    reference's fp16 key, csrc/topk_select.cu:26-31) are widened exactly to fp32, which keeps their order and ties."""
    logits = np.asarray(logits, dtype=np.float32)
    rows, Lc = logits.shape
    out = np.full((rows, K), -1, dtype=np.int32)
    for r in range(rows):
        n = max(0, min(int(ctx[r]), Lc))
        if n == 0:
            continue
        kv = okey(logits[r, :n]).astype(np.int64)
        order = np.lexsort((np.arange(n), -kv))[:K]            # primary: key desc, secondary: column asc
        vals = logits[r, order]
        sel = np.where(np.isinf(vals), -1, order).astype(np.int32)
        out[r, :sel.size] = sel
    return out


def topk_local(logits, ctx, rank, P, kl):
    """fast_topk.local (dotsnote/engine/arcstats_pkg/arcstats/fast_topk.py:52-66; csrc/topk_select.cu:1-13, :75-201):
    valid columns j < ceil((ctx - rank) / P) clipped to Lc; the top kl (key okey desc, lower column first) in
    ascending column order -> pk [rows, 2 kl] float32 = [values | positions j * P + rank (int32 bits)]; short rows
    padded with -inf at positions s * P + rank."""
    logits = np.asarray(logits, dtype=np.float32)
    rows, Lc = logits.shape
    pk = np.zeros((rows, 2 * kl), dtype=np.float32)
    pos = pk[:, kl:].view(np.int32)
    for r in range(rows):
        c = int(ctx[r])
        n = min(Lc, (c - rank + P - 1) // P) if c > rank else 0
        kv = okey(logits[r, :n]).astype(np.int64)
        chosen = np.sort(np.lexsort((np.arange(n), -kv))[:kl])    # the selection, then ascending columns
        m = chosen.size
        pk[r, :m] = logits[r, chosen]
        pos[r, :m] = chosen * P + rank
        pk[r, m:kl] = -np.inf
        pos[r, m:kl] = np.arange(m, kl) * P + rank
    return pk


def topk_merge(allp, n, P, kl, kk, topk_tokens):
    """fast_topk.merge (fast_topk.py:69-78; csrc/topk_select.cu:203-244): per row the top kk of the P * kl gathered
    candidates by (key desc, concatenation index asc) -> positions, -1 for +-inf values and slots >= kk."""
    a = np.asarray(allp, dtype=np.float32).reshape(P, n, 2 * kl)
    out = np.full((n, topk_tokens), -1, dtype=np.int32)
    for r in range(n):
        vals = a[:, r, :kl].reshape(-1)
        poss = a[:, r, kl:].copy().view(np.int32).reshape(-1)
        kv = okey(vals).astype(np.int64)
        order = np.lexsort((np.arange(vals.size), -kv))[:kk]
        out[r, :order.size] = np.where(np.isinf(vals[order]), -1, poss[order])
    return out


def rows_from_topk(topk_pos, req, block_table, block_size, stride_rows=None):
    """rows = block_table[req, p // bs] * stride_rows + p % bs for p >= 0 inside the table and a block id >= 0,
    else -1 (vLLM triton_convert_req_index_to_global_index semantics at dsa_sm89.py:314-315, :467-469)."""
    stride_rows = block_size if stride_rows is None else stride_rows
    tp = np.asarray(topk_pos, dtype=np.int64)
    bt = np.asarray(block_table, dtype=np.int64)
    out = np.full(tp.shape, -1, dtype=np.int64)
    for t in range(tp.shape[0]):
        for k in range(tp.shape[1]):
            p = tp[t, k]
            if p < 0 or p // block_size >= bt.shape[1]:
                continue
            b = bt[req[t], p // block_size]
            if b >= 0:
                out[t, k] = b * stride_rows + p % block_size
    return out.astype(np.int32)


def compact_stage(rows, sidx):
    """(rows [tot], sidx [M, K]) -> (sel = rows of the sorted distinct selected positions, sidx2 into sel)
    (dotsnote/engine/arcstats_pkg/arcstats/dsa_sm89.py:27-35)."""
    sidx = np.asarray(sidx, dtype=np.int64)
    v = sidx >= 0
    u, inv = np.unique(sidx[v], return_inverse=True)
    sidx2 = np.full(sidx.shape, -1, dtype=np.int64)
    sidx2[v] = inv
    return np.asarray(rows)[u], sidx2.astype(np.int32)


def gather(src, rows):
    """dst[i] = src[rows[i]] for 0 <= rows[i] < R, zero row otherwise (sparse_offload.py:293-306)."""
    src = np.asarray(src)
    rows = np.asarray(rows, dtype=np.int64)
    ok = (rows >= 0) & (rows < src.shape[0])
    out = np.zeros((rows.shape[0], src.shape[1]), dtype=src.dtype)
    out[ok] = src[rows[ok]]
    return out


def tier_split(idx, rowmap, R):
    """Per token: valid host rows with a cache line -> HBM list (line), others -> host list (row), stable order,
    -1 padded (hit / miss resolution of the row cache, offload_fill.py:204-248)."""
    idx = np.asarray(idx, dtype=np.int64)
    T, K = idx.shape
    hbm = np.full((T, K), -1, dtype=np.int32)
    host = np.full((T, K), -1, dtype=np.int32)
    hc = np.zeros(T, dtype=np.int32)
    sc = np.zeros(T, dtype=np.int32)
    for t in range(T):
        a, b = [], []
        for h in idx[t]:
            if 0 <= h < R:
                (a.append(int(rowmap[h])) if rowmap[h] >= 0 else b.append(int(h)))
        hbm[t, :len(a)] = a
        host[t, :len(b)] = b
        hc[t], sc[t] = len(a), len(b)
    return hbm, hc, host, sc


# ------------------------------------------------------------------------------------------------ W-way row cache
def wcache_step(tag, rr, idx, R, W):
    """One decode step of the W-way set-associative row cache (dotsnote/engine/arcstats_pkg/arcstats/sparse_offload.py
    :677-770, composed by _sa_prefill :1595-1622), for the outputs that do not depend on the order in which the
    device's atomics serve the misses. tag [C] (-1 empty), rr [S] (S = C / W), idx [T, K] host rows (valid iff in
    [0, R)). Row h belongs to set h % S. Returns a dict:
      hits       number of valid entries whose row is in a line of its set before the step;
      pinned     lines hit (never replaced in this step);
      misses     distinct valid rows not cached, in ascending order;
      placed     {set: lines that receive misses} = the first min(m, u) unpinned ways counted from rr[set] (m misses
                 and u unpinned ways in the set);
      spills     number of misses that find no way: sum over sets of max(0, m - u);
      rr_next    rr[set] + min(m, W) mod W;
      content    {set: sorted tags after the step} for every set with m <= u (the placed lines then hold exactly the
                 set's misses)."""
    tag = np.asarray(tag, dtype=np.int64)
    rr = np.asarray(rr, dtype=np.int64)
    C = tag.shape[0]
    S = C // W
    pinned, miss, hits = set(), set(), 0
    for h in np.asarray(idx, dtype=np.int64).reshape(-1):
        if not (0 <= h < R):
            continue
        st = int(h % S)
        ways = [st * W + w for w in range(W) if tag[st * W + w] == h]
        if ways:
            hits += 1
            pinned.add(ways[0])
        else:
            miss.add(int(h))
    by_set = {}
    for h in sorted(miss):
        by_set.setdefault(h % S, []).append(h)
    placed, content, spills = {}, {}, 0
    rr_next = rr.copy()
    for st, rows in by_set.items():
        free = [st * W + (int(rr[st]) + j) % W for j in range(W) if st * W + (int(rr[st]) + j) % W not in pinned]
        m, u = len(rows), len(free)
        placed[st] = free[:min(m, u)]
        spills += max(0, m - u)
        rr_next[st] = (rr[st] + min(m, W)) % W
        if m <= u:
            t = tag.copy()
            t[placed[st]] = rows
            content[st] = sorted(t[st * W:(st + 1) * W].tolist())
    return {"hits": hits, "pinned": pinned, "misses": sorted(miss), "placed": placed, "spills": spills,
            "rr_next": rr_next, "content": content}


def wcache_set2(h, S):
    """Second candidate set of host row h under two-choice placement (dotsnote/engine/arcstats_pkg/arcstats/
    offload_fill.py:136-138: ((h * 2654435761) >> 12) % S, in 64-bit integers)."""
    return ((int(h) * 2654435761) >> 12) % S


def wcache_step2(tag, rr, idx, R, W):
    """The order-independent part of a step with two-choice placement (offload_fill.py:141-165 scan with P2: an
    entry that misses its first set h % S looks in wcache_set2(h, S), a hit there pins that line): hits, pinned lines
    and the distinct missing rows (ascending), as dicts like wcache_step's."""
    tag = np.asarray(tag, dtype=np.int64)
    C = tag.shape[0]
    S = C // W
    pinned, miss, hits = set(), set(), 0
    for h in np.asarray(idx, dtype=np.int64).reshape(-1):
        if not (0 <= h < R):
            continue
        line = -1
        for st in (int(h % S), wcache_set2(h, S)):
            ways = [st * W + w for w in range(W) if tag[st * W + w] == h]
            if ways:
                line = ways[0]
                break
        if line >= 0:
            hits += 1
            pinned.add(line)
        else:
            miss.add(int(h))
    return {"hits": hits, "pinned": pinned, "misses": sorted(miss), "S": S, "W": W}


def wcache_verify2(model, tag, rr, tag_after, rr_after, spills):
    """Conditions every outcome of a two-choice step satisfies, whatever order the device's atomics serve the misses
    in (offload_fill.py:255-293 alloc with P2, advance sparse_offload.py:747-752); returns the violated ones (empty =
    consistent). Each miss takes ticket k = cnt[s]++ in its first set s and the k-th unpinned way counted from rr[s];
    if k reaches the set's unpinned ways u_s it takes a ticket in its second set the same way, and past that it
    spills. So, with p_s the lines of set s that changed and T_s its tickets (its own misses plus the misses not placed
    in their first set whose second set is s): pinned lines keep their rows; a changed line holds a miss, in one of
    that miss's two sets, each miss at most once; the changed lines of s are its first p_s unpinned ways from rr[s];
    p_s = min(T_s, u_s); a miss outside its first set needs that set full (p = u), a spilled miss both sets full;
    spills = misses - placed; rr_after[s] = rr[s] + min(T_s, W) mod W."""
    S, W = model["S"], model["W"]
    tag = np.asarray(tag, dtype=np.int64)
    ta = np.asarray(tag_after, dtype=np.int64)
    rr = np.asarray(rr, dtype=np.int64)
    misses = set(model["misses"])
    bad = []
    if any(ta[l] != tag[l] for l in model["pinned"]):
        bad.append("pinned line replaced")
    changed = np.nonzero(ta != tag)[0].tolist()
    where = {}
    for l in changed:
        h = int(ta[l])
        if h not in misses:
            bad.append(f"line {l} holds {h}, not a miss of the step")
            continue
        if l // W not in (h % S, wcache_set2(h, S)):
            bad.append(f"row {h} placed outside its two sets")
        if h in where:
            bad.append(f"row {h} placed twice")
        where[h] = l // W
    if spills != len(misses) - len(where):
        bad.append(f"spills {spills} != misses {len(misses)} - placed {len(where)}")
    pin = model["pinned"]
    unp = [[s * W + (int(rr[s]) + j) % W for j in range(W) if s * W + (int(rr[s]) + j) % W not in pin]
           for s in range(S)]
    p = np.zeros(S, dtype=np.int64)
    for l in changed:
        p[l // W] += 1
    tickets = np.zeros(S, dtype=np.int64)
    for h in misses:
        s1 = h % S
        tickets[s1] += 1
        if where.get(h) != s1:                         # its first ticket failed
            tickets[wcache_set2(h, S)] += 1
            if p[s1] != len(unp[s1]):
                bad.append(f"row {h} left its first set {s1} with a free way")
            if h not in where and p[wcache_set2(h, S)] != len(unp[wcache_set2(h, S)]):
                bad.append(f"row {h} spilled with a free way in its second set")
    for s in range(S):
        if sorted(l for l in changed if l // W == s) != sorted(unp[s][:p[s]]):
            bad.append(f"set {s}: replaced lines are not its first {p[s]} unpinned ways from rr")
        if p[s] != min(tickets[s], len(unp[s])):
            bad.append(f"set {s}: {p[s]} lines placed for {tickets[s]} tickets and {len(unp[s])} free ways")
        if int(rr_after[s]) != (int(rr[s]) + min(int(tickets[s]), W)) % W:
            bad.append(f"set {s}: rr {int(rr_after[s])} after {tickets[s]} tickets from {int(rr[s])}")
    return bad


# ------------------------------------------------------------------------------------------------ MLA absorbed matmuls
def bmm_fp8_weights(codes, scales, scale_k):
    """bf16 values (as float64) of block-scaled FP8 weights W[n][j][k] = bf16(fp32(e4m3(code) * S)), S =
    scales[n][j][k // 128] (scale_k) else scales[n][k][j // 128] (dotsnote/engine/arcstats_pkg/arcstats/mla_fp8.py:
    46-52: (w.to(float32) * s).to(bfloat16))."""
    c = np.asarray(codes, dtype=np.uint8)
    N, J, K = c.shape
    s = np.asarray(scales, dtype=np.float32)
    if scale_k:
        S = np.repeat(s, 128, axis=2)[:, :, :K]
    else:
        S = np.repeat(s, 128, axis=2)[:, :, :J].transpose(0, 2, 1)
    prod = (e4m3_decode(c).astype(np.float32) * S.astype(np.float32)).astype(np.float32)
    return bf16_bits_to_f32(f32_to_bf16_bits(prod)).astype(np.float64)


def bmm_fp8(a, codes, scales, scale_k):
    """C[n][b][j] = sum_k A[n][b][k] * W[n][j][k] (mla_fp8.py:20-57), A the bf16 values, float64 result."""
    W = bmm_fp8_weights(codes, scales, scale_k)
    return np.einsum("nbk,njk->nbj", np.asarray(a, dtype=np.float64), W)


def topk_overlap(sets):
    """Top-k overlap of L layers' selections (dotsnote/engine/arcstats_pkg/arcstats/index_share.py:109-130): sets
    int [L, n, K] (-1 = none) -> hits [L, L, n] (hits[a, b, i] = number of entries x >= 0 of sets[b, i] with x in
    sets[a, i], counted with multiplicity in b; diagonal 0) and nvalid [L, n] (entries >= 0)."""
    s = np.asarray(sets, dtype=np.int64)
    L, n, K = s.shape
    hits = np.zeros((L, L, n), dtype=np.int64)
    nvalid = (s >= 0).sum(axis=2)
    for i in range(n):
        for a in range(L):
            A = s[a, i][s[a, i] >= 0]
            for b in range(L):
                if a == b:
                    continue
                B = s[b, i][s[b, i] >= 0]
                hits[a, b, i] = int(np.isin(B, A).sum())
    return hits, nvalid


def shuffle_layout(rows, bs):
    """132-byte key rows [R, 132] (R a multiple of bs) -> vLLM's paged SHUFFLE cache [R / bs, bs * 132]: in block b,
    code d of key t at (t // 16) * 16 * 128 + (t % 16) * 16 + (d // 16) * 256 + d % 16, its fp32 scale at
    bs * 128 + 4 t (dotsnote/engine/arcstats_pkg/arcstats/dsa_sm89.py:63-66)."""
    rows = np.asarray(rows, dtype=np.uint8)
    nb = rows.shape[0] // bs
    out = np.zeros((nb, bs * KEYROW), dtype=np.uint8)
    t = np.arange(bs)[:, None]
    d = np.arange(128)[None, :]
    off = (t // 16) * 2048 + (t % 16) * 16 + (d // 16) * 256 + d % 16
    for b in range(nb):
        blk = rows[b * bs:(b + 1) * bs]
        out[b, off] = blk[:, :128]
        out[b, bs * 128:] = blk[:, 128:132].reshape(-1)
    return out


def shuffle_rows(cache, bs):
    """Inverse of shuffle_layout: [nb, bs * 132] -> [nb * bs, 132]."""
    cache = np.asarray(cache, dtype=np.uint8).reshape(-1, bs * KEYROW)
    nb = cache.shape[0]
    rows = np.zeros((nb * bs, KEYROW), dtype=np.uint8)
    t = np.arange(bs)[:, None]
    d = np.arange(128)[None, :]
    off = (t // 16) * 2048 + (t % 16) * 16 + (d // 16) * 256 + d % 16
    for b in range(nb):
        rows[b * bs:(b + 1) * bs, :128] = cache[b, off]
        rows[b * bs:(b + 1) * bs, 128:132] = cache[b, bs * 128:].reshape(bs, 4)
    return rows


def index_key_write_shuffle(k_bits, slots, cache, bs, ue8m0=False):
    """The indexer key write into the SHUFFLE cache: the same per-key quantization as index_key_write (P = 1),
    stored at slot = block * bs + t in the layout of shuffle_layout."""
    rows = shuffle_rows(cache, bs)
    index_key_write(k_bits, slots, rows, P=1, rank=0, ue8m0=ue8m0)
    cache[...] = shuffle_layout(rows, bs).reshape(cache.shape)
    return cache


def paged_ctx(seq_lens, next_n):
    """Per logits row r = b * next_n + j: (request b, visible keys) as paged_mqa_logits_triton reads them
    (dsa_sm89.py:46-53): seq_lens[b] - (next_n - 1 - j), or seq_lens[b, j] when seq_lens is 2-D."""
    sl = np.asarray(seq_lens, dtype=np.int64)
    B = sl.shape[0]
    req = np.repeat(np.arange(B), next_n)
    j = np.tile(np.arange(next_n), B)
    ctx = sl.reshape(-1) if sl.ndim == 2 else sl[req] - (next_n - 1 - j)
    return req, ctx


def paged_mqa_logits(q, cache, w, seq_lens, block_table, bs, max_model_len):
    """paged_mqa_logits_triton (dsa_sm89.py:41-94): q [B, next_n, H, D] values, cache [nb, bs * 132] SHUFFLE bytes,
    w [B * next_n, H] -> [B * next_n, max_model_len] float64, -inf outside each row's context (no clamp)."""
    q = np.asarray(q, dtype=np.float64)
    B, nn, H, D = q.shape
    req, ctx = paged_ctx(seq_lens, nn)
    return index_logits(q.reshape(B * nn, H, D), w, shuffle_rows(cache, bs), block_table, bs, req, ctx,
                        max_model_len, clamp=np.inf)


def mqa_logits(q, codes, scales, w, ks, ke):
    """mqa_logits_triton (dsa_sm89.py:97-133): q [M, H, D] values, codes [N, 128] e4m3, scales [N] fp32, w [M, H],
    valid keys ks[m] <= n < ke[m] -> [M, N] float64, -inf elsewhere (no clamp)."""
    q = np.asarray(q, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    M, N = q.shape[0], codes.shape[0]
    kc = e4m3_decode(np.asarray(codes, dtype=np.uint8)).astype(np.float64)
    sc = np.asarray(scales, dtype=np.float32).astype(np.float64)
    out = np.full((M, N), -np.inf)
    for m in range(M):
        n = np.arange(max(0, int(ks[m])), min(N, int(ke[m])))
        if n.size:
            out[m, n] = (w[m] @ np.maximum(q[m] @ kc[n].T, 0.0)) * sc[n]
    return out


def mtp_union(idx, T, ql, cu, nreq, R, nmax, gmax=6):
    """The request's union of MTP top-k rows (dotsnote/engine/arcstats_pkg/arcstats/csrc/offload_attn.cu:586-698):
    for request r, tokens t0 .. t0 + G - 1 (G = min(t1 - t0, 6)), entries at position j * topk + k; each valid row
    (0 <= row < R) once, with mask = OR of 1 << j over the tokens j that selected it, ordered by mask descending
    then by the position of its first occurrence. Returns (u [nreq, nmax] int (-1 padded), mk [nreq, nmax] uint8
    (0 where padded), cnt [nreq])."""
    idx = np.asarray(idx)
    topk = idx.shape[1]
    u = np.full((nreq, nmax), -1, dtype=np.int64)
    mk = np.zeros((nreq, nmax), dtype=np.uint8)
    cnt = np.zeros(nreq, dtype=np.int64)
    for r in range(nreq):
        t0 = int(cu[r]) if cu is not None else min(r * ql, T)
        t1 = int(cu[r + 1]) if cu is not None else min(t0 + ql, T)
        G = min(max(t1 - t0, 0), gmax)
        mask, first = {}, {}
        for j in range(G):
            for k in range(topk):
                h = int(idx[t0 + j, k])
                if 0 <= h < R:
                    mask[h] = mask.get(h, 0) | (1 << j)
                    first.setdefault(h, j * topk + k)
        order = sorted(mask, key=lambda h: (-mask[h], first[h]))
        cnt[r] = len(order)
        u[r, :len(order)] = order
        mk[r, :len(order)] = [mask[h] for h in order]
    return u, mk, cnt
