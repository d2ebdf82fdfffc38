"""Random valid ggml Q4_K / Q6_K / Q8_0 matrices for the matrix-vector tests:
random code, scale and min bytes, with the fp16 block scales set to finite,
moderate values (random bytes there could be Inf/NaN)."""
import numpy as np

Q8_0, Q4_K, Q6_K = 8, 12, 14
BLOCK = {Q4_K: 144, Q6_K: 210}


def random_matrix(rng, dtype, n_rows, n_in, scale=1.0):
    """scale multiplies the fp16 super-block scales (1.0: |w| up to ~4)."""
    if dtype == Q8_0:
        # codes in [-127, 127] (what ggml's quantizers write), d per 32 weights
        nb = n_rows * (n_in // 32)
        raw = np.empty((nb, 34), np.uint8)
        raw[:, 2:] = rng.integers(-127, 128, size=(nb, 32)).astype(np.int8).view(np.uint8)
        d = (rng.uniform(1e-3, 3e-2, nb) * scale).astype(np.float16)
        raw[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        return raw.reshape(-1)
    nb = n_rows * (n_in // 256)
    raw = rng.integers(0, 256, size=(nb, BLOCK[dtype]), dtype=np.uint8)
    if dtype == Q4_K:
        d = (rng.uniform(2e-4, 4e-3, nb) * scale).astype(np.float16)
        dmin = (rng.uniform(1e-4, 2e-3, nb) * scale).astype(np.float16)
        raw[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        raw[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    else:
        d = (rng.uniform(1e-5, 2e-4, nb) * scale).astype(np.float16)
        raw[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    return raw.reshape(-1)
