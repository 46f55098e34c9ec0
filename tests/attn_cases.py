"""Case builders shared by the GPU parity tests.

The prefill corpus is the reference's (engine/src/gpu_attention_validation.rs): geometry
12/3/64, context 1024 (table stride 64), 3 layers with layer 1 under test, counter-hash
values (:47-86), physical pages from a seeded Fisher-Yates shuffle assigned round-robin
across requests (:125-148), finite poison in unused slots and future pages (:149-183),
and the fixed case list of :431-509. Pools hold fp16 (the allowed layout change), so K/V
are the fp16 rounding of the reference's f32 values and the oracle reads the same bits.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

import oracle

HEADS, KV_HEADS, HD = 12, 3, 64
D, KD = HEADS * HD, KV_HEADS * HD
CONTEXT, STRIDE, LAYERS, LAYER = 1024, 64, 3, 1
SENTINEL = -12345.25
SEED = 20260908


@dataclass
class Slice:
    id: int
    start: int
    len: int


@dataclass
class Case:
    name: str
    slices: list
    seed: int
    profile: int


def q_value(case, s, pos, h, d):
    p = case.profile
    if p == 1:
        return 0.0
    if p == 2:
        return 0.0 if h % 4 == 0 else oracle.value(s.id, pos, h, d, 19) * [1.0, 0.125, 8.0, -16.0][h % 4]
    if p == 3:
        return [16.0, -16.0, 1.0, -1.0][h % 4] if d == 0 else 0.0
    return oracle.value(s.id, pos, h, d, 19) * [0.25, 1.0, -2.0, 4.0][h % 4]


def k_value(case, id_, pos, h, d):
    if case.profile == 3 and d == 0:
        return pos * 0.125 + h * 0.375
    return oracle.value(id_, pos, h, d, 31)


def homogeneous(name, count, length, start, seed):
    return Case(name, [Slice(i, start, length) for i in range(count)], seed, 2)


def cases(seed=SEED):
    out = []
    for p in [0, 1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257, 511, 512,
              513, 1023]:
        out.append(homogeneous(f"boundary-{p}", 1, 1, p, seed + p))
    for start in [1, 15, 16, 17, 63, 64, 127, 128, 255, 512, 960]:
        out.append(homogeneous(f"offset-{start}", 3, 64, start, seed + start))
    for length in [1, 16, 32, 64, 128, 256, 512, 768, 941, 1024]:
        out.append(homogeneous(f"single-{length}", 1, length, 0, seed + length))
    for count, length in [(16, 16), (8, 32), (4, 64), (4, 128), (4, 256), (8, 128), (2, 512)]:
        out.append(homogeneous(f"{count}x{length}", count, length, 0, seed + count))
    for profile in range(4):
        out.append(Case(f"ragged-profile-{profile}",
                        [Slice(0, 0, 17), Slice(1, 15, 33), Slice(2, 255, 129), Slice(3, 512, 257)],
                        seed + profile, profile))
    return out


def fuzz_cases(n=64, seed=SEED):
    """The reference's fuzz corpus (gpu_attention_validation.rs:564-586; 64 rounds at seed
    20260908 by default, main.rs:216-219): 1..16 requests per case, each with a length drawn
    from the remaining context budget (at most 257) and a random start, ids round * 16 + i,
    the case seed and Q profile round % 4, all from the xorshift stream (:40-45)."""
    stream = _Xorshift(max(seed, 1))
    out = []
    for rnd in range(n):
        count = 1 + stream.next() % 16
        remaining = CONTEXT
        slices = []
        for i in range(count):
            length = 1 + stream.next() % min(remaining - (count - i - 1), 257)
            start = stream.next() % (CONTEXT - length + 1)
            slices.append(Slice(rnd * 16 + i, start, length))
            remaining -= length
        out.append(Case(f"fuzz-{rnd}", slices, stream.next(), rnd % 4))
    return out


class _Xorshift:
    """xorshift64 13/7/17 (gpu_attention_validation.rs:40-45) through the oracle's
    orc_xorshift, one value at a time."""

    def __init__(self, state):
        import ctypes

        self._st = ctypes.c_uint64(state)

    def next(self) -> int:
        import ctypes

        return int(oracle.lib().orc_xorshift(ctypes.byref(self._st)))


def _values(case, id_, n_pos):
    """[n_pos, KV_HEADS, HD] K (salt 31; profile 3 ramps d=0) and V (salt 47), float32."""
    k = oracle.value_grid(id_, 0, n_pos, KV_HEADS, HD, 31)
    v = oracle.value_grid(id_, 0, n_pos, KV_HEADS, HD, 47)
    if case.profile == 3:
        pos = np.arange(n_pos, dtype=np.float32)[:, None]
        k[:, :, 0] = pos * np.float32(0.125) + np.arange(KV_HEADS, dtype=np.float32) * np.float32(0.375)
    return k, v


def _queries(case, s):
    """[len, HEADS*HD] query rows of slice s (gpu_attention_validation.rs:63-77)."""
    n = s.len
    p = case.profile
    if p == 1:
        return np.zeros((n, HEADS * HD), np.float32)
    if p == 3:
        q = np.zeros((n, HEADS, HD), np.float32)
        q[:, :, 0] = np.array([16.0, -16.0, 1.0, -1.0], np.float32)[np.arange(HEADS) % 4]
        return q.reshape(n, -1)
    base = oracle.value_grid(s.id, s.start, n, HEADS, HD, 19)
    mult = [1.0, 0.125, 8.0, -16.0] if p == 2 else [0.25, 1.0, -2.0, 4.0]
    scale = np.array(mult, np.float32)[np.arange(HEADS) % 4]
    if p == 2:
        scale = np.where(np.arange(HEADS) % 4 == 0, np.float32(0.0), scale).astype(np.float32)
    return (base * scale[None, :, None]).reshape(n, -1).astype(np.float32)


@dataclass
class Fixture:
    case: Case
    q: np.ndarray            # [rows, D] float32
    k_pool: np.ndarray       # uint16 fp16 bits (K order)
    v_pool: np.ndarray       # uint16 fp16 bits (V block-transposed)
    tables: np.ndarray       # [requests, STRIDE] int32
    owners: np.ndarray
    positions: np.ndarray
    segments: np.ndarray     # [requests, 4] int32
    rows: int
    max_chunk: int


def fixture(case: Case, poison_future: bool = False) -> Fixture:
    pages = [-(-min(s.start + s.len + 16, CONTEXT) // 16) for s in case.slices]
    total = sum(pages)
    mapping = oracle.shuffle(max(case.seed, 1), total)
    tables = np.full((len(case.slices), STRIDE), -1, np.int32)
    nxt = 0
    for page in range(max(pages)):
        for r, count in enumerate(pages):
            if page < count:
                tables[r, page] = mapping[nxt]
                nxt += 1
    n_elem = total * LAYERS * 16 * KD
    k_ref = np.full(n_elem, np.float32(99.75), np.float32)      # reference element order
    v_ref = np.full(n_elem, np.float32(-87.125), np.float32)
    q, owners, positions, segments = [], [], [], []
    packed = 0
    for r, s in enumerate(case.slices):
        segments.append([packed, s.len, s.start, r])
        kv_k, kv_v = _values(case, s.id, pages[r] * 16)
        for pos in range(pages[r] * 16):
            phys = tables[r, pos // 16]
            off = ((phys * LAYERS + LAYER) * 16 + pos % 16) * KD
            future = poison_future and pos >= s.start + s.len
            k_ref[off:off + KD] = 123.75 if future else kv_k[pos].reshape(-1)
            v_ref[off:off + KD] = -987.25 if future else kv_v[pos].reshape(-1)
        owners.extend([r] * s.len)
        positions.extend(range(s.start, s.start + s.len))
        q.append(_queries(case, s))
        packed += s.len
    k_bits = oracle.f32_to_f16_bits(k_ref)
    v_bits = oracle.v_blocks_from_reference(oracle.f32_to_f16_bits(v_ref), KD)
    tables_clean = np.where(tables < 0, 0, tables).astype(np.int32)
    return Fixture(case, np.concatenate(q).astype(np.float32), k_bits, v_bits, tables_clean,
                   np.array(owners, np.int32), np.array(positions, np.int32),
                   np.array(segments, np.int32), packed, max(s.len for s in case.slices))


def oracle_out(fx: Fixture, q=None) -> np.ndarray:
    q = fx.q if q is None else q
    return oracle.attention_paged_rows(q, fx.k_pool, fx.v_pool, fx.tables, fx.positions + 1,
                                       table_index=fx.owners, n_head=HEADS, n_kv_head=KV_HEADS,
                                       head_dim=HD, table_stride=STRIDE, n_layer=LAYERS,
                                       layer=LAYER)


def oracle_abs_v(fx: Fixture, q=None) -> np.ndarray:
    """The same attention over |V| (fp16 sign bits cleared): per output element the weighted
    mean sum_i w_i |v_i| of its row's softmax weights, which bounds what rounding the weights
    can move it by (gates.element_gate's P16 term)."""
    q = fx.q if q is None else q
    return oracle.attention_paged_rows(q, fx.k_pool, fx.v_pool & np.uint16(0x7FFF), fx.tables,
                                       fx.positions + 1, table_index=fx.owners, n_head=HEADS,
                                       n_kv_head=KV_HEADS, head_dim=HD, table_stride=STRIDE,
                                       n_layer=LAYERS, layer=LAYER)


def random_pools(rng, n_pages, n_layer, kv_dim, scale=1.0):
    n = n_pages * n_layer * 16 * kv_dim
    k = oracle.f32_to_f16_bits(rng.standard_normal(n).astype(np.float32) * scale)
    v = oracle.f32_to_f16_bits(rng.standard_normal(n).astype(np.float32))
    return k, v


def disjoint_tables(rng, n_pages, lens, stride):
    perm = rng.permutation(n_pages).astype(np.int32)
    tables = np.zeros((len(lens), stride), np.int32)
    cur = 0
    for b, n in enumerate(lens):
        need = -(-int(n) // 16)
        tables[b, :need] = perm[cur:cur + need]
        cur += need
    assert cur <= n_pages
    return tables
