"""GPU parity of the argmax LM head (ds_argmax_matvec_bf16, ds_hip_argmax_bf16) against the oracle's
or_argmax_bf16, index bit-exact. Shapes cover every ring depth of the one-row-per-lane kernel
(in_dim/64 odd, even, a multiple of 4), ragged vocabularies, reference thread counts whose row
chunks are or are not whole groups of 4 (the latter take the general kernel), and planted rows:
exact ties (lowest index wins), NaN products (never chosen), -inf rows and an all-excluded head
(index 0)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

BF16_NAN = 0x7FC0
BF16_NEG_INF = 0xFF80

# (in_dim, vocab, reference threads)
SHAPES = [
    (64, 4, 1),
    (64, 256, 4),
    (128, 1000, 5),
    (128, 1016, 5),
    (192, 4100, 1),
    (256, 2048, 16),
    (320, 260, 1),
    (1280, 5000, 8),
    (1280, 20480, 16),
]


def eligible(in_dim, vocab, T):
    chunk = vocab if T <= 1 else -(-vocab // T)
    return in_dim % 64 == 0 and all(min(chunk, vocab - s) % 4 == 0 for s in range(0, vocab, chunk))


def planted(B, in_dim, vocab, seed, kind):
    W = B.normal_bf16(vocab * in_dim, seed, 0.02).reshape(vocab, in_dim)
    x = B.normal_f32(in_dim, seed + 1)
    if kind == "ties" and vocab >= 8:
        big = B.f32_to_bf16_rne(np.sign(x) * 0.5)
        a, b = vocab // 3, vocab - 2
        W[a] = big
        W[b] = big
        W[1] = B.f32_to_bf16_rne(np.sign(x) * 0.25)
    elif kind == "nan_best" and vocab >= 8:
        W[vocab // 2] = B.f32_to_bf16_rne(np.sign(x) * 0.5)
        W[vocab // 2, in_dim // 2] = BF16_NAN
        W[vocab // 4] = B.f32_to_bf16_rne(np.sign(x) * 0.4)
        W[vocab - 1, :] = BF16_NEG_INF
    elif kind == "all_excluded":
        W[:, :] = BF16_NEG_INF
        x = np.abs(x) + 0.5
    return np.ascontiguousarray(W), np.ascontiguousarray(x.astype(np.float32))


@pytest.mark.parametrize("kind", ["random", "ties", "nan_best", "all_excluded"])
@pytest.mark.parametrize("in_dim,vocab,T", SHAPES)
def test_lm_argmax_vs_oracle(dev, B, in_dim, vocab, T, kind):
    if kind == "all_excluded" and vocab > 5000:
        pytest.skip("covered at the smaller shapes")
    L = dev.load()
    W, x = planted(B, in_dim, vocab, 1000 + in_dim + vocab, kind)
    val = np.zeros(1, np.float32)
    want = B.oracle().or_argmax_bf16(x, W, in_dim, vocab, T, val.ctypes.data_as(B.C.POINTER(B.C.c_float)))
    if kind == "all_excluded":
        assert want == 0
    try:
        L.ds_set_threads(T)
        got_host = L.ds_argmax_matvec_bf16(x, W, in_dim, vocab)
        Wd = dev.DeviceBuffer.from_array(W)
        xd = dev.DeviceBuffer.from_array(x)
        idx = dev.DeviceBuffer(4)
        dev.check(L.ds_hip_argmax_bf16(idx.ptr, xd.ptr, Wd.ptr, in_dim, vocab), "argmax")
        dev.check(L.ds_hip_sync(), "sync")
        got_dev = int(idx.to_array(np.int32)[0])
    finally:
        L.ds_set_threads(1)
    path = "fast" if eligible(in_dim, vocab, T) else "general"
    assert got_host == want, (path, got_host, want)
    assert got_dev == want, (path, got_dev, want)


def test_config4_226_steps(dev, B):
    """Config 4: the 129280 x 1280 bf16 head, 226 sequential steps, each on a fresh seeded
    f32[1280] ~ N(0, 1) input, 16 reference threads: every index equal to the oracle's (the oracle's
    226 argmaxes run on host threads; ctypes releases the GIL)."""
    from concurrent.futures import ThreadPoolExecutor
    L = dev.load()
    V, H, N = 129280, 1280, 226
    W = B.normal_bf16(V * H, 4242, 0.02)
    xs = np.stack([B.normal_f32(H, 40000 + s) for s in range(N)])
    Wd = dev.DeviceBuffer.from_array(W)
    xd = dev.DeviceBuffer.from_array(xs)
    idx = dev.DeviceBuffer(4 * N)
    try:
        L.ds_set_threads(16)
        for s in range(N):
            dev.check(L.ds_hip_argmax_bf16(idx.ptr + 4 * s, xd.ptr + 4 * H * s, Wd.ptr, H, V), "argmax")
        dev.check(L.ds_hip_sync(), "sync")
    finally:
        L.ds_set_threads(1)
    got = idx.to_array(np.int32)
    with ThreadPoolExecutor(8) as ex:
        want = np.array(list(ex.map(lambda s: B.oracle().or_argmax_bf16(xs[s], W, H, V, 16, None), range(N))))
    print(f"config 4: {int(np.sum(got == want))}/{N} indices equal")
    assert np.array_equal(got, want)


def test_config4_226_steps_bounded_head(dev, B):
    """Config 4 through the drop-in ds_argmax_matvec_bf16 (host pointers) at 16 threads, the path
    that serves the head from its int8 copy with exact bounds (k_lm_q8_argmax, the kernel the bench
    times): 226 steps on fresh seeded inputs, every index equal to or_argmax_bf16's."""
    from concurrent.futures import ThreadPoolExecutor
    L = dev.load()
    V, H, N = 129280, 1280, 226
    W = B.normal_bf16(V * H, 4343, 0.02)
    xs = np.stack([B.normal_f32(H, 50000 + s) for s in range(N)])
    try:
        L.ds_set_threads(16)
        got = np.array([L.ds_argmax_matvec_bf16(xs[s], W, H, V) for s in range(N)])
        assert L.ds_hip_argmax_int8_copy(W.ctypes.data) == 1  # the bounded head served these calls
    finally:
        L.ds_hip_weights_changed(W.ctypes.data)
        L.ds_set_threads(1)
    with ThreadPoolExecutor(8) as ex:
        want = np.array(list(ex.map(lambda s: B.oracle().or_argmax_bf16(xs[s], W, H, V, 16, None), range(N))))
    print(f"config 4, bounded head: {int(np.sum(got == want))}/{N} indices equal")
    assert np.array_equal(got, want)


def test_lm_argmax_config5_head(dev, B):
    """The full 129280 x 1280 head of config 5, 16 reference threads (chunks of 8080 rows)."""
    L = dev.load()
    V, H = 129280, 1280
    W = B.normal_bf16(V * H, 4242, 0.02).reshape(V, H)
    for s in range(3):
        x = B.normal_f32(H, 777 + s)
        want = B.oracle().or_argmax_bf16(x, W, H, V, 16, None)
        try:
            L.ds_set_threads(16)
            got = L.ds_argmax_matvec_bf16(x, W, H, V)
        finally:
            L.ds_set_threads(1)
        assert got == want, (s, got, want)


def test_weights_changed_in_place_are_seen(dev, B):
    """The host API registers host weights once (keyed by address); an in-place edit of one row is
    announced with ds_hip_weights_changed and must then change the answer; a new array at another
    address is uploaded on its own."""
    L = dev.load()
    in_dim, vocab = 128, 4096
    W, x = planted(B, in_dim, vocab, 77, "random")
    first = L.ds_argmax_matvec_bf16(x, W, in_dim, vocab)
    assert first == B.oracle().or_argmax_bf16(x, W, in_dim, vocab, 1, None)
    target = vocab - 5 if first != vocab - 5 else 7
    W[target] = B.f32_to_bf16_rne(np.sign(x) * 0.5)
    assert L.ds_hip_weights_changed(W.ctypes.data) == 1
    assert L.ds_argmax_matvec_bf16(x, W, in_dim, vocab) == target
    assert L.ds_hip_weights_changed(W.ctypes.data) == 1
    assert L.ds_hip_weights_changed(W.ctypes.data) == 0  # nothing registered any more
    W2 = W.copy()
    W2[target] = W2[first]
    assert L.ds_argmax_matvec_bf16(x, W2, in_dim, vocab) == min(first, target)
    # ds_bf16_dot_row reads the row from the registered head: equal to the oracle's sequential chain
    v = L.ds_bf16_dot_row(x, W2, in_dim, target)
    assert np.float32(v).view(np.uint32) == np.float32(B.oracle().or_bf16_dot_row(x, W2, in_dim, target)).view(np.uint32)


def test_argmax_never_returns_an_index_outside_the_rows(dev, B):
    """Invalid arguments (or a device error) give 0, a row the reference's caller may read
    (ds_moe_decoder.c:1041-1043), never -1."""
    L = dev.load()
    W, x = planted(B, 128, 256, 78, "random")
    assert L.ds_argmax_matvec_bf16(x, W, 0, 256) == 0
    assert L.ds_argmax_matvec_bf16(x, W, 128, 0) == 0
