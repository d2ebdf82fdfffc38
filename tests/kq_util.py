"""Random valid ggml Q4_K / Q6_K matrices for the matrix-vector tests: random
code, scale and min bytes, with the fp16 super-block scales set to finite,
moderate values (random bytes there could be Inf/NaN)."""
import numpy as np

Q4_K, Q6_K = 12, 14
BLOCK = {Q4_K: 144, Q6_K: 210}


def random_matrix(rng, dtype, n_rows, n_in, scale=1.0):
    """scale multiplies the fp16 super-block scales (1.0: |w| up to ~4)."""
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
