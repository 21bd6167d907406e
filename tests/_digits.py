"""The grouped kernels' digit image of an activation row, restated with
numpy (the layout of lpk::dimage_bytes): per 32-column sub-group g, 16-bit
fixed point against the sub-group's largest magnitude m, xq = rint(x *
(32639 / m)) in fp32, split into int8 digits hi = (xq + 128) >> 8 and lo =
xq - 256 hi, stored in MFMA operand order (byte t of half h holds column
16h + 8 (t >> 3) + 2 (t & 3) + ((t >> 2) & 1)); then (0, -8 sum xq) as int32
and sigma = m / 32639 as f32.  Sub-groups with m below 1e-30 are zero."""
import numpy as np

DIGIT_COL = np.array([16 * h + 8 * (t >> 3) + 2 * (t & 3) + ((t >> 2) & 1) for h in range(2) for t in range(16)])


def ngp(cols: int) -> int:
    return 4 * (((cols >> 5) + 3) >> 2)


def digit_image(row: np.ndarray) -> np.ndarray:
    """uint8 image of one f32 row."""
    cols = row.size
    n = ngp(cols)
    v = np.zeros(n * 32, np.float32)
    v[:cols] = row
    v = v.reshape(n, 32)
    m = np.abs(v).max(axis=1)
    live = m >= np.float32(1e-30)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = np.where(live, np.float32(32639.0) / m, np.float32(0)).astype(np.float32)
        sigma = np.where(live, m / np.float32(32639.0), np.float32(0)).astype(np.float32)
    xq = np.rint((v * inv[:, None]).astype(np.float32)).astype(np.int64)
    hi = (xq + 128) >> 8
    lo = xq - 256 * hi
    img = np.zeros(76 * n, np.uint8)
    img[: 32 * n] = hi[:, DIGIT_COL].astype(np.int8).view(np.uint8).ravel()
    img[32 * n: 64 * n] = lo[:, DIGIT_COL].astype(np.int8).view(np.uint8).ravel()
    seeds = np.zeros((n, 2), np.int32)
    seeds[:, 1] = -8 * xq.sum(axis=1)
    img[64 * n: 72 * n] = seeds.view(np.uint8).ravel()
    img[72 * n:] = sigma.view(np.uint8)
    return img


def decode_image(img: np.ndarray, cols: int):
    """(x reconstructed from the digits, sigma per sub-group, seeds [n, 2])."""
    n = ngp(cols)
    hi = img[: 32 * n].view(np.int8).reshape(n, 32).astype(np.int64)
    lo = img[32 * n: 64 * n].view(np.int8).reshape(n, 32).astype(np.int64)
    xq = np.zeros((n, 32), np.int64)
    xq[:, DIGIT_COL] = 256 * hi + lo
    seeds = img[64 * n: 72 * n].view(np.int32).reshape(n, 2)
    sigma = img[72 * n:].view(np.float32)
    return (xq * sigma[:, None].astype(np.float64)).ravel()[:cols], sigma, seeds, xq


def assert_digit_images(images: np.ndarray, x: np.ndarray) -> None:
    """The device's images of the rows of x: equal to the restatement byte for
    byte, and each value within half a digit step of x (sigma / 2, plus
    |xq| times the rounding of sigma against 1 / inv: 32639 * 2^-23 sigma)."""
    T, cols = x.shape
    for t in range(T):
        want = digit_image(x[t])
        assert np.array_equal(images[t], want), t
        rec, sigma, seeds, xq = decode_image(images[t], cols)
        sg = np.repeat(sigma.astype(np.float64), 32)[:cols]
        assert np.all(np.abs(rec - x[t].astype(np.float64)) <= 0.505 * sg + 1e-30), t
        assert np.array_equal(seeds[:, 1], -8 * xq.sum(axis=1)) and not seeds[:, 0].any(), t
        assert np.abs(xq).max() <= 32639
