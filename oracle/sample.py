"""Oracle for the fused token sampler (test infrastructure: only tests/, the smoke check and
bench.py's CPU baseline use it; the product path never calls it).

What it restates.  The reference samples every row's next token with one batched call
(chat.py:103-107): probs = softmax(logits.float() / temperature), then torch.multinomial(probs, 1).
For one sample per row, torch.multinomial draws by the exponential race: with E_v ~ Exp(1)
independent, token = argmax_v probs_v / E_v (ATen's multinomial, n_sample == 1 branch).  In log
space the softmax normaliser cancels:

    token = argmax_v ( logit_v / temperature - ln E_v ),   E_v = -ln U_v,  U_v ~ Uniform(0, 1)

which is the Gumbel-max form.  temperature <= 0 means greedy: argmax_v logit_v.  Ties go to the
lowest index; NaN logits never win; a row with no finite-or-+inf candidate gets -1.

Where the uniforms come from (the kernel's own choice, not torch's stream): Philox4x32-10
(Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC 2011), keyed by the
64-bit seed, counter (v // 4, row, offset low 32 bits, offset high 32 bits); output word v % 4 of
that block is vocabulary entry v's uniform, U = (2 * (x >> 9) + 1) * 2^-24, which lies in
[2^-24, 1 - 2^-24] and is exact in fp32.

Pinned by tests/test_sample.py: the Random123 known-answer vectors for philox4x32-10, an
independent scalar Philox, the sample distribution against softmax probabilities (chi-square),
greedy limits and planted mistakes.
"""
import numpy as np

PHILOX_M0 = 0xD2511F53
PHILOX_M1 = 0xCD9E8D57
PHILOX_W0 = 0x9E3779B9
PHILOX_W1 = 0xBB67AE85
MASK32 = 0xFFFFFFFF


def philox4x32(c0, c1, c2, c3, k0, k1, rounds=10):
    """Vectorised Philox4x32: counters (c0..c3) and key (k0, k1) as uint32 arrays or scalars;
    returns the four output words as uint32 arrays."""
    c = [np.asarray(x, dtype=np.uint64) & MASK32 for x in (c0, c1, c2, c3)]
    k0 = np.asarray(k0, dtype=np.uint64) & MASK32
    k1 = np.asarray(k1, dtype=np.uint64) & MASK32
    for r in range(rounds):
        if r:
            k0 = (k0 + PHILOX_W0) & MASK32
            k1 = (k1 + PHILOX_W1) & MASK32
        p0 = c[0] * np.uint64(PHILOX_M0)
        p1 = c[2] * np.uint64(PHILOX_M1)
        hi0, lo0 = p0 >> np.uint64(32), p0 & MASK32
        hi1, lo1 = p1 >> np.uint64(32), p1 & MASK32
        c = [hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0]
    return [x.astype(np.uint32) for x in c]


def uniforms(batch, vocab, seed, offset):
    """U [batch, vocab] float64 (exactly the fp32 values the kernel forms)."""
    v = np.arange(vocab, dtype=np.uint64)
    rows = np.arange(batch, dtype=np.uint64)[:, None]
    g = (v // 4)[None, :]
    words = philox4x32(g, rows, offset & MASK32, (offset >> 32) & MASK32,
                       seed & MASK32, (seed >> 32) & MASK32)
    w = np.stack(words, axis=-1)                                # [batch, vocab, 4]
    x = np.take_along_axis(w, (v % 4).astype(np.int64)[None, :, None].repeat(batch, 0), -1)[..., 0]
    return (2.0 * (x >> 9).astype(np.float64) + 1.0) * 2.0 ** -24


def scores(logits, temperature, seed, offset):
    """The race scores logit / T - ln(-ln U) in float64 (greedy: the logits themselves)."""
    lg = np.asarray(logits, dtype=np.float64)
    if temperature <= 0:
        return lg.copy()
    u = uniforms(lg.shape[0], lg.shape[1], seed, offset)
    return lg / np.float64(np.float32(temperature)) - np.log(-np.log(u))


def sample(logits, temperature, seed, offset):
    """One token id per row of logits [batch, vocab] (int64, -1 for a row with no candidate)."""
    s = scores(logits, temperature, seed, offset)
    s = np.where(np.isnan(s), -np.inf, s)
    out = np.argmax(s, axis=1).astype(np.int64)
    out[np.all(s == -np.inf, axis=1)] = -1
    return out
