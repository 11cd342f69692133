"""Shared helpers for the tests: seeded inputs, tolerances, reference-style PRNG."""
import numpy as np


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


def xorshift_vec(n: int, seed: int) -> np.ndarray:
    """The reference tests' PRNG (kernels.rs:1311-1321): xorshift32 mapped to ~U(-1, 1) in f32."""
    s = seed & 0xFFFFFFFF
    out = np.empty(n, np.float32)
    for i in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out[i] = (np.float32(s) / np.float32(4294967295.0) - np.float32(0.5)) * np.float32(2.0)
    return out


def normal(shape, seed, std=1.0) -> np.ndarray:
    return (np.random.default_rng(seed).standard_normal(shape) * std).astype(np.float32)


def bits_equal(a, b) -> bool:
    """Bitwise equality of f32 arrays, treating any two NaNs as equal."""
    a = np.ascontiguousarray(a, np.float32).ravel()
    b = np.ascontiguousarray(b, np.float32).ravel()
    same = a.view(np.uint32) == b.view(np.uint32)
    both_nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(same | both_nan))


def boundary_router(E: int, H: int, k: int, x: np.ndarray):
    """A router whose last top-k place only the sequential fp32 fold decides (kernels.rs:113-124).

    Experts a = 1 and b = 2 have the same exact logit 1 + 2^-18 (a: 1 then sixty-four 2^-24 terms;
    b: the sixty-four 2^-24 terms then 1), so any sum taken more accurately than the fold ties them
    and orders a (the lower id) first. The fold gives a exactly 1 (each 2^-24 after the leading 1 is
    half an ulp and rounds to even) and b 1 + 2^-18 (its small terms add exactly before the 1), so b
    takes the last place. k - 1 experts (ids 3, 6, 9, ...) rank above both with logits 1.5 + j/16;
    every other expert's logit is 0. x (one token, changed in place) gets ones in its first 65
    entries, the only ones the rows use. Returns (router [E, H], a, b, the k - 1 higher ids)."""
    m = 64
    x[:m + 1] = 1.0
    router = np.zeros((E, H), np.float32)
    d = np.float32(2.0 ** -24)
    hi = [3 + 3 * j for j in range(k - 1)]
    assert hi[-1] < E
    for j, e in enumerate(hi):
        router[e, 0] = np.float32(1.5 + j / 16)
    a, b = 1, 2
    router[a, 0] = 1.0
    router[a, 1:m + 1] = d
    router[b, :m] = d
    router[b, m] = 1.0
    return router, a, b, hi


def tied_boundary_router(E: int, H: int, k: int, x: np.ndarray, n_tied: int = 5):
    """A router whose last top-k place n_tied experts contest with the same exact logit 1 + 2^-18:
    tied expert i has 1.0 at position p_i = 64 i / (n_tied - 1) of its first 65 entries and 2^-24
    at the other 64. Any sum more accurate than the fold ties them (midpoint order: lower id
    first); the sequential fp32 fold (kernels.rs:113-124) adds the p_i small terms exactly, then
    the 1 (exact for even p_i), and every later 2^-24 is half an ulp that rounds to even, so it gives
    1 + 2^-23 m_i with m_i = p_i / 2 rounded up to even. The fold thus ranks the tied experts in
    the opposite order to their ids: the highest id takes the place. k - 1 experts (ids 3, 6, 9,
    ...) rank above with logits 1.5 + j/16; every other logit is 0. x (one token, changed in place)
    gets ones in its first 65 entries. Returns (router [E, H], tied ids, their fold values, the
    k - 1 higher ids)."""
    m = 64
    x[:m + 1] = 1.0
    router = np.zeros((E, H), np.float32)
    d = np.float32(2.0 ** -24)
    hi = [3 + 3 * j for j in range(k - 1)]
    tied = [e for e in range(1, E) if e % 3 != 0][:n_tied]
    assert hi[-1] < E and len(tied) == n_tied
    for j, e in enumerate(hi):
        router[e, 0] = np.float32(1.5 + j / 16)
    folds = []
    for i, e in enumerate(tied):
        p = m * i // (n_tied - 1)
        router[e, :m + 1] = d
        router[e, p] = 1.0
        mi = p // 2 + (p // 2) % 2 if p % 2 == 0 else None
        assert mi is not None, "positions must be even"
        folds.append(np.float32(1.0 + mi * 2.0 ** -23))
    return router, tied, folds, hi


def write_safetensors(path, tensors, metadata=None, raw_header=None):
    """Writes a safetensors file: tensors is a list of (name, dtype, shape, bytes) in data order.
    raw_header (bytes), when given, replaces the JSON header (for malformed-header tests)."""
    import json
    header, data = {}, bytearray()
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, dtype, shape, b in tensors:
        b = bytes(b)
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [len(data), len(data) + len(b)]}
        data += b
    hb = raw_header if raw_header is not None else json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(len(hb).to_bytes(8, "little"))
        f.write(hb)
        f.write(data)


class HipGraph:
    """A HIP graph captured from a stream (the library's) through the runtime's C API."""

    def __init__(self, stream: int):
        import ctypes as C
        self.C = C
        self.hip = C.CDLL("libamdhip64.so.7")
        self.stream = C.c_void_p(stream)
        self.graph, self.exec = C.c_void_p(), C.c_void_p()

    def _ok(self, rc, what):
        if rc:
            raise RuntimeError(f"{what} -> {rc}")

    def begin(self):
        self._ok(self.hip.hipStreamBeginCapture(self.stream, 1), "hipStreamBeginCapture")  # thread-local mode

    def end(self):
        self._ok(self.hip.hipStreamEndCapture(self.stream, self.C.byref(self.graph)), "hipStreamEndCapture")
        self._ok(self.hip.hipGraphInstantiate(self.C.byref(self.exec), self.graph, None, None, self.C.c_size_t(0)),
                 "hipGraphInstantiate")

    def launch(self):
        self._ok(self.hip.hipGraphLaunch(self.exec, self.stream), "hipGraphLaunch")

    def destroy(self):
        if self.exec:
            self.hip.hipGraphExecDestroy(self.exec)
        if self.graph:
            self.hip.hipGraphDestroy(self.graph)
        self.exec = self.graph = self.C.c_void_p()
