"""Model-level pieces on the CPU: the FNV-1a hash pinned to its published
test vectors, the eval oracle's cross-entropy pinned to torch's
cross_entropy as the reference calls it (grafting.hip:527-532), and the
certify gates (deploy/certify.sh:28-59)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O


def test_fnv1a64_known_answers():
    # published FNV-1a 64-bit test vectors (with the published basis)
    h0 = O.FNV_BASIS_PUBLISHED
    assert O.fnv1a64(b"", h0) == 0xcbf29ce484222325
    assert O.fnv1a64(b"a", h0) == 0xaf63dc4c8601ec8c
    assert O.fnv1a64(b"foobar", h0) == 0x85944171f73967e8
    # the reference's basis constant (grafting.hip:505) is that number with
    # its last digit dropped; the eval hash starts from it
    assert O.FNV_BASIS == O.FNV_BASIS_PUBLISHED // 10 and O.fnv1a64(b"") == O.FNV_BASIS


def test_eval_oracle_ce_matches_torch_cross_entropy():
    rng = np.random.default_rng(1)
    B, T, V = 3, 7, 300
    x = O.bf16_round(rng.normal(0, 4, (B, T, V)).astype(np.float32))
    ids = rng.integers(0, V, (B, T)).astype(np.int32)
    st = O.eval_stats(x, ids)
    lt = torch.tensor(x)[:, :T - 1].permute(0, 2, 1).contiguous()
    ce = torch.nn.functional.cross_entropy(lt, torch.tensor(ids[:, 1:].astype(np.int64)), reduction="mean")
    assert st["count"] == B * (T - 1)
    assert st["total_nll"] / st["count"] == pytest.approx(ce.item(), rel=1e-6)
    assert st["logits_sum"] == pytest.approx(float(x.astype(np.float64).sum()), rel=1e-12)


def test_eval_hash_is_order_and_value_sensitive():
    rng = np.random.default_rng(2)
    x = O.bf16_round(rng.normal(0, 1, (1, 4, 16)).astype(np.float32))
    ids = np.zeros((1, 4), np.int32)
    for ref in (True, False):
        h = O.eval_stats(x, ids, reference_hash=ref)["logits_hash"]
        y = x.copy()
        y[0, 2, 5] = np.nextafter(y[0, 2, 5], np.float32(np.inf))
        assert O.eval_stats(y, ids, reference_hash=ref)["logits_hash"] != h
        z = x[:, ::-1].copy()
        assert O.eval_stats(z, ids, reference_hash=ref)["logits_hash"] != h
    # row form. One row of 16: sixteen one-element chunks, each hashed from
    # the basis, the chunk hashes' bytes hashed in order, then that row
    # hash's 8 bytes
    fb = lambda a: a.astype("<f4").tobytes()
    r = O.eval_stats(x[:, :1], ids[:, :1], reference_hash=False)["logits_hash"]
    chunks = b"".join(O.fnv1a64(fb(x[0, 0, c:c + 1])).to_bytes(8, "little") for c in range(16))
    assert r == O.fnv1a64(O.fnv1a64(chunks).to_bytes(8, "little"))
    # 20 elements: ten chunks of two, six empty chunks (an empty chunk hashes to the basis)
    w = O.bf16_round(rng.normal(0, 1, 20).astype(np.float32))
    chunks = b"".join(O.fnv1a64(fb(w[2 * c:2 * c + 2])).to_bytes(8, "little") for c in range(10))
    chunks += O.FNV_BASIS.to_bytes(8, "little") * 6
    assert O.eval_row_hash(w) == O.fnv1a64(chunks)


def test_certify_gates():
    from glt_amd import ops
    A = {"ce": 2.0, "logits_hash": 7}
    B = {"ce": 1.5, "logits_hash": 8}
    C = {"ce": 1.51, "logits_hash": 9}
    r = ops.certify(A, B, C, dict(A))
    assert r["pass"] == 1 and r["content"] == "A_STANDALONE_DELTAS"
    assert ops.certify(A, B, {"ce": 1.6, "logits_hash": 9}, dict(A))["gate_bake_equal"] == 0
    assert ops.certify(A, {"ce": 2.0, "logits_hash": 8}, {"ce": 2.0, "logits_hash": 9}, dict(A))["content"] == \
        "B_BAKED_MISLABEL_SUSPECT"
    assert ops.certify(A, B, C, {"ce": 2.0, "logits_hash": 6})["gate_reload_equal"] == 0


def _reference_hash_loop(logits, h=O.FNV_BASIS):
    """The reference's loop written out (grafting.hip:536-546): for b, t, v
    the f32 logit's four bytes in memory order, h ^= byte; h *= prime."""
    B, T, V = logits.shape
    for b in range(B):
        for t in range(T):
            for v in range(V):
                for byte in np.float32(logits[b, t, v]).tobytes():   # little-endian on x86-64
                    h = ((h ^ byte) * 1099511628211) % (1 << 64)
    return h


def test_eval_reference_hash_is_the_sequential_byte_chain():
    """The oracle's reference hash (through the C FNV) equals the reference's
    loop written out, continues from any start (the reference chains its
    eval batches), and its C FNV agrees with the published vectors."""
    rng = np.random.default_rng(3)
    x = O.bf16_round(rng.normal(0, 3, (2, 3, 37)).astype(np.float32))
    assert O.eval_hash_reference(x) == _reference_hash_loop(x)
    h1 = O.eval_hash_reference(x[:1])
    assert O.eval_hash_reference(x[1:], h1) == O.eval_hash_reference(x)
    assert O.eval_stats(x, np.zeros((2, 3), np.int32))["logits_hash"] == _reference_hash_loop(x)
    assert O.fnv1a64_c(b"foobar", O.FNV_BASIS_PUBLISHED) == 0x85944171f73967e8
    data = rng.integers(0, 256, 1000).astype(np.uint8).tobytes()
    assert O.fnv1a64_c(data, 12345) == O.fnv1a64(data, 12345)


def _parallel_hash(bits16, h, chunks):
    """The decomposition the GPU computes, restated on the CPU: the low byte
    of the state is a chain of its own (low nibble first, then high nibble,
    each a 16-state map per chunk composed in order), after which each chunk
    is the affine map h -> h * P^(4n) + B mod 2^64."""
    P, M64 = 1099511628211, (1 << 64) - 1

    def run8(c, s):
        for w in c:
            s = (s * P * P) & 0xFF
            s = ((s ^ (int(w) & 0xFF)) * P) & 0xFF
            s = ((s ^ (int(w) >> 8)) * P) & 0xFF
        return s

    def run64(c, hh):
        for w in c:
            for byte in (0, 0, int(w) & 0xFF, int(w) >> 8):
                hh = ((hh ^ byte) * P) & M64
        return hh

    n = -(-len(bits16) // chunks)
    cs = [bits16[i * n:(i + 1) * n] for i in range(chunks)]
    lo, s_lo = h & 15, []
    for c in cs:
        s_lo.append(lo)
        lo = [run8(c, i) & 15 for i in range(16)][lo]
    hi, s8 = (h >> 4) & 15, []
    for c, l in zip(cs, s_lo):
        s8.append((hi << 4) | l)
        hi = [run8(c, (i << 4) | l) >> 4 for i in range(16)][hi]
    for c, s in zip(cs, s8):
        a = pow(P, 4 * len(c), 1 << 64)
        h = (h * a + (run64(c, s) - s * a)) & M64
    return h


def test_parallel_hash_decomposition_reproduces_the_chain():
    rng = np.random.default_rng(4)
    for n, chunks in ((1, 1), (50, 7), (333, 16), (64, 64)):
        x = O.bf16_round(rng.normal(0, 2, n).astype(np.float32))
        bits = O.f32_to_bf16_bits(x)
        for h in (O.FNV_BASIS, int(rng.integers(0, 2 ** 63)) * 2 + 1):
            assert _parallel_hash(bits, h, chunks) == O.eval_hash_reference(x, h)


def _bit_plane_runs(wa, wb):
    """The low-nibble pass as the GPU runs it (bit planes): bit i of plane j
    is bit j of run i's nibble, chunk A's 16 runs in the low 16 bits and
    chunk B's in the high 16 bits of each 32-bit plane. Per logit pair
    (16-bit patterns a, b): 9 s flips bit 3 by bit 0, XOR with a logit bit
    is a XOR with that bit spread over its half, 3 s = s + 2 s is a ripple
    carry over the planes."""
    M = 0xFFFFFFFF

    def half_mask(w, k):
        return (0xFFFF if (w >> k) & 1 else 0) | (0xFFFF0000 if (w >> (16 + k)) & 1 else 0)

    def x3(p0, p1, p2, p3):
        c1, t = p1 & p0, p2 ^ p1
        c2 = (t & c1) | (~t & p2 & M)
        return p0, p1 ^ p0, t ^ c1, p3 ^ p2 ^ c2

    p = (0xAAAAAAAA, 0xCCCCCCCC, 0xF0F0F0F0, 0xFF00FF00)   # run i starts at nibble i
    for a, b in zip(wa, wb):
        w = int(a) | (int(b) << 16)
        p0, p1, p2, p3 = p
        p3 ^= p0 ^ half_mask(w, 3)
        p = x3(p0 ^ half_mask(w, 0), p1 ^ half_mask(w, 1), p2 ^ half_mask(w, 2), p3)
        p = x3(*(pj ^ half_mask(w, 8 + j) for j, pj in enumerate(p)))
    runs = lambda off: [sum(((p[j] >> (off + i)) & 1) << j for j in range(4)) for i in range(16)]
    return runs(0), runs(16)


def test_bit_plane_low_nibble_pass_is_the_chain():
    """The GPU's bit-plane form of the low-nibble pass gives, for every start
    nibble and both chunks of a pair, the low nibble that the reference's
    byte chain reaches (bytes 0, 0, lo, hi per logit)."""
    rng = np.random.default_rng(5)
    P = 1099511628211

    def chain(s, ws):
        for w in ws:
            for byte in (0, 0, int(w) & 0xFF, int(w) >> 8):
                s = ((s ^ byte) * P) & 0xFF
        return s & 15

    for n in (0, 1, 7, 40):
        wa = rng.integers(0, 1 << 16, n)
        wb = rng.integers(0, 1 << 16, n)
        ra, rb = _bit_plane_runs(wa, wb)
        assert ra == [chain(i, wa) for i in range(16)]
        assert rb == [chain(i, wb) for i in range(16)]
