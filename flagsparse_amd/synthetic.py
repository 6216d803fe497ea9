"""Seeded synthetic CSR inputs for the benchmark configurations.

Generation runs on whatever device the caller names (the GPU for the full
sizes, the CPU for small test cases) with a torch.Generator seeded per
config, so a run and its CPU baseline see the same matrix.

Configs (BASELINE.json "configs"):
  C1 uniform_rows      4096 x 4096, exactly 16 distinct sorted cols/row, f32/i32
  C2 stencil27         27-point stencil on an n^3 grid (boundary rows
                       truncated), off-diagonal U(0.5,1.5), diagonal 27, f64/i32
  C3 powerlaw          row length min(Zipf(2.0) + 9, 50000) (clipped Zipf(2)
                       alone has mean 6.93; the +9 shift gives mean ~15.93
                       and keeps the exponent-2 tail), uniform distinct sorted
                       cols, f32, i32 or i64
  C4 uniform_rows      1,048,576^2, 32 cols/row, f32/i32, dense B 1M x 64
  C5 rmat              R-MAT scale 21, 16 edges/vertex, (a,b,c,d) =
                       (0.57,0.19,0.19,0.05), duplicates removed, f32 U(0,1)
                       values, i64 indices, dense B 2^21 x 256 N(0,1)
"""


import torch


def _gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def _uniform(n, lo, hi, dtype, device, g):
    real = dtype
    if dtype == torch.complex64:
        real = torch.float32
    elif dtype == torch.complex128:
        real = torch.float64
    t = torch.rand(n, dtype=real, device=device, generator=g) * (hi - lo) + lo
    if real is not dtype:
        im = torch.rand(n, dtype=real, device=device, generator=g) * (hi - lo) + lo
        t = torch.complex(t, im)
    return t


def _indptr_from_lengths(lengths, dtype):
    indptr = torch.zeros(lengths.numel() + 1, dtype=torch.int64, device=lengths.device)
    indptr[1:] = torch.cumsum(lengths.to(torch.int64), 0)
    return indptr.to(dtype)


def distinct_sorted_columns(lengths, n_cols, g):
    """Per-row columns drawn uniformly without replacement, sorted per row.

    Draw with replacement, sort by (row, col), redraw the later copy of any
    duplicate, repeat until every row is duplicate-free.
    """
    device = lengths.device
    n_rows = lengths.numel()
    lengths = lengths.to(torch.int64)
    if int(lengths.max().item() if n_rows else 0) > n_cols:
        raise ValueError("row length exceeds n_cols")
    rows = torch.repeat_interleave(torch.arange(n_rows, device=device, dtype=torch.int64), lengths)
    cols = torch.randint(0, n_cols, (rows.numel(),), device=device, generator=g, dtype=torch.int64)
    # Rows filling more than a quarter of the columns: a sorted prefix of a
    # random permutation (rejection would converge slowly there).
    dense_rows = torch.nonzero(lengths * 4 > n_cols).flatten().tolist()
    if dense_rows:
        starts = torch.cumsum(lengths, 0) - lengths
        for r in dense_rows:
            s0, ln = int(starts[r]), int(lengths[r])
            perm = torch.randperm(n_cols, device=device, generator=g)[:ln]
            cols[s0:s0 + ln] = torch.sort(perm)[0]
    for _ in range(64):
        key, _ = torch.sort(rows * n_cols + cols)
        cols = key - rows * n_cols
        if key.numel() < 2:
            break
        dup = torch.nonzero(key[1:] == key[:-1]).flatten() + 1
        if dup.numel() == 0:
            break
        cols[dup] = torch.randint(0, n_cols, (dup.numel(),), device=device, generator=g, dtype=torch.int64)
    else:
        raise RuntimeError("could not draw distinct columns")
    return cols


def uniform_rows(n_rows, n_cols, per_row, dtype=torch.float32, index_dtype=torch.int32, device="cpu", seed=0,
                 lo=-1.0, hi=1.0):
    """CSR with exactly `per_row` distinct sorted uniform columns per row (C1, C4)."""
    g = _gen(device, seed)
    lengths = torch.full((n_rows,), per_row, dtype=torch.int64, device=device)
    cols = distinct_sorted_columns(lengths, n_cols, g)
    data = _uniform(cols.numel(), lo, hi, dtype, device, g)
    return data, cols.to(index_dtype), _indptr_from_lengths(lengths, index_dtype), (n_rows, n_cols)


def stencil27(n=128, dtype=torch.float64, index_dtype=torch.int32, device="cpu", seed=0):
    """27-point stencil on an n^3 grid, row i = (x*n + y)*n + z (C2).

    Neighbours at offsets in {-1,0,1}^3 inside the grid; columns ascend in
    offset order.  Off-diagonal U(0.5, 1.5), diagonal 27.
    """
    g = _gen(device, seed)
    ar = torch.arange(n, device=device, dtype=torch.int64)
    X, Y, Z = torch.meshgrid(ar, ar, ar, indexing="ij")
    X, Y, Z = X.reshape(-1), Y.reshape(-1), Z.reshape(-1)
    row = (X * n + Y) * n + Z
    cols, masks = [], []
    for dx in (-1, 0, 1):
        for dy in (-1, 0, 1):
            for dz in (-1, 0, 1):
                ok = (X + dx >= 0) & (X + dx < n) & (Y + dy >= 0) & (Y + dy < n) & (Z + dz >= 0) & (Z + dz < n)
                cols.append(row + (dx * n + dy) * n + dz)
                masks.append(ok)
    cols = torch.stack(cols, 1)
    masks = torch.stack(masks, 1)
    lengths = masks.sum(1)
    col_flat = cols[masks]
    diag = (col_flat == torch.repeat_interleave(row, lengths))
    data = _uniform(col_flat.numel(), 0.5, 1.5, dtype, device, g)
    data[diag] = 27.0
    return data, col_flat.to(index_dtype), _indptr_from_lengths(lengths, index_dtype), (n**3, n**3)


def zipf_lengths(n_rows, exponent=2.0, shift=9, clip=50000, device="cpu", g=None):
    """min(Zipf(exponent) + shift, clip) via the inverse CDF of the zeta law."""
    kmax = clip - shift  # Zipf values >= kmax all clip to `clip`
    k = torch.arange(1, kmax, dtype=torch.float64, device=device)
    pmf = k.pow(-exponent)
    zeta = sum(1.0 / (i**exponent) for i in range(1, 200001)) + 1.0 / ((exponent - 1) * 200000 ** (exponent - 1))
    cdf = torch.cumsum(pmf, 0) / zeta
    u = torch.rand(n_rows, dtype=torch.float64, device=device, generator=g)
    z = torch.searchsorted(cdf, u, right=True) + 1  # values 1..kmax (kmax == clipped tail)
    return torch.clamp(z + shift, max=clip)


def powerlaw(n=4194304, dtype=torch.float32, index_dtype=torch.int32, device="cpu", seed=0, exponent=2.0,
             shift=9, clip=50000):
    """C3: Zipf row lengths, uniform distinct sorted columns, U(-1,1) values."""
    g = _gen(device, seed)
    lengths = zipf_lengths(n, exponent, shift, min(clip, max(shift + 2, n // 8)), device, g)
    cols = distinct_sorted_columns(lengths, n, g)
    data = _uniform(cols.numel(), -1.0, 1.0, dtype, device, g)
    return data, cols.to(index_dtype), _indptr_from_lengths(lengths, index_dtype), (n, n)


def rmat(scale=21, edge_factor=16, a=0.57, b=0.19, c=0.19, dtype=torch.float32, index_dtype=torch.int64,
         device="cpu", seed=0):
    """C5: R-MAT edges, duplicates removed, sorted CSR, U(0,1) values."""
    g = _gen(device, seed)
    n = 1 << scale
    m = edge_factor * n
    row = torch.zeros(m, dtype=torch.int64, device=device)
    col = torch.zeros(m, dtype=torch.int64, device=device)
    for _ in range(scale):
        u = torch.rand(m, device=device, generator=g)
        rbit = (u >= a + b).to(torch.int64)
        cbit = (((u >= a) & (u < a + b)) | (u >= a + b + c)).to(torch.int64)
        row = row * 2 + rbit
        col = col * 2 + cbit
    key = torch.unique(row * n + col, sorted=True)
    row = key // n
    col = key - row * n
    lengths = torch.bincount(row, minlength=n)
    data = _uniform(key.numel(), 0.0, 1.0, dtype, device, g)
    return data, col.to(index_dtype), _indptr_from_lengths(lengths, index_dtype), (n, n)


def dense(rows, cols, dtype, device="cpu", seed=0, dist="uniform"):
    """Dense operand: U(-1,1) or N(0,1) (complex: independent parts)."""
    g = _gen(device, seed)
    real = {torch.complex64: torch.float32, torch.complex128: torch.float64}.get(dtype, dtype)
    if dist == "normal":
        t = torch.randn((rows, cols), dtype=real, device=device, generator=g)
        if real is not dtype:
            t = torch.complex(t, torch.randn((rows, cols), dtype=real, device=device, generator=g))
        return t
    t = torch.rand((rows, cols), dtype=real, device=device, generator=g) * 2 - 1
    if real is not dtype:
        t = torch.complex(t, torch.rand((rows, cols), dtype=real, device=device, generator=g) * 2 - 1)
    return t


def vector(n, dtype, device="cpu", seed=0):
    return dense(n, 1, dtype, device, seed).reshape(-1)


def random_csr(n_rows, n_cols, density, dtype=torch.float32, index_dtype=torch.int32, device="cpu", seed=0,
               empty_row_every=0, long_rows=()):
    """Small irregular test matrix: Bernoulli(density) pattern, optional
    forced-empty rows and forced long rows (row, length)."""
    g = _gen(device, seed)
    lengths = torch.distributions.Binomial(n_cols, torch.full((n_rows,), float(density), device=device)).sample()
    lengths = lengths.to(torch.int64)
    if empty_row_every:
        lengths[::empty_row_every] = 0
    for r, ln in long_rows:
        lengths[r] = min(int(ln), n_cols)
    cols = distinct_sorted_columns(lengths, n_cols, g) if n_rows else torch.empty(0, dtype=torch.int64)
    data = _uniform(cols.numel(), -1.0, 1.0, dtype, device, g)
    return data, cols.to(index_dtype), _indptr_from_lengths(lengths, index_dtype), (n_rows, n_cols)


def bytes_spmv(nnz, n_rows, n_cols, val_bytes, idx_bytes, ptr_bytes):
    """Algorithmic HBM bytes of one SpMV: A once, x once, y once."""
    return nnz * (val_bytes + idx_bytes) + (n_rows + 1) * ptr_bytes + n_cols * val_bytes + n_rows * val_bytes


def bytes_spmm(nnz, m, k, n, val_bytes, idx_bytes, ptr_bytes):
    """Algorithmic HBM bytes of one SpMM: A once, B once, C once."""
    return nnz * (val_bytes + idx_bytes) + (m + 1) * ptr_bytes + k * n * val_bytes + m * n * val_bytes


def flops_spmv(nnz, complex_values=False):
    return (8 if complex_values else 2) * nnz


def flops_spmm(nnz, n, complex_values=False):
    return (8 if complex_values else 2) * nnz * n
