"""Root-of-unity conventions of the reference, for building RNS requests.

The RNS ABI takes explicit forward ring roots. These helpers pick them the way
the reference does: the smallest candidate c in [2, 2^20) whose c^((q-1)/n) has
exact order n (src/reference.cpp:564-582), and for the negacyclic ring the
crypto benchmark's psi whose square is that n-th root
(benchmarks/crypto_ntt/crypto_ntt_bench.cu:273-290).
"""


def primitive_root(log_n, q):
    n = 1 << log_n
    if (q - 1) % n:
        raise ValueError("modulus - 1 is not divisible by the requested length")
    for c in range(2, 1 << 20):
        w = pow(c, (q - 1) // n, q)
        if pow(w, n, q) == 1 and pow(w, n // 2, q) != 1:
            return w
    raise ValueError("no primitive power-of-two root below 2^20")


def psi_for_root(log_n, q, root):
    first = primitive_root(log_n + 1, q)
    if first * first % q == root:
        return first
    order = 2 << log_n
    for c in range(2, 1 << 20):
        psi = pow(c, (q - 1) // order, q)
        if pow(psi, order, q) == 1 and pow(psi, order // 2, q) != 1 and psi * psi % q == root:
            return psi
    raise ValueError("no 2n-th root squares to the given root")
