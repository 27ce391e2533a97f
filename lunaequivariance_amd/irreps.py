"""e3nn-compatible irreducible-representation labels.

Mirrors the parsing and layout rules of the reference's ``src/o3/irreps.py``
(``Irrep`` :17-82, ``_MulIr`` :85-106, ``Irreps`` :109-242): an irrep is
``(l, p)`` with dimension ``2l+1``; ``"16x1o"`` is 16 copies laid out
copy-major, so component ``m`` of copy ``u`` sits at ``offset + u*(2l+1) + m``.
"""

from __future__ import annotations

from typing import Iterable


class Irrep(tuple):
    """Degree ``l`` and parity ``p`` (``+1`` even, ``-1`` odd)."""

    def __new__(cls, l, p=None):
        if p is None:
            if isinstance(l, Irrep):
                return l
            if isinstance(l, MulIr):
                return l.ir
            if isinstance(l, str):
                text = l.strip()
                try:
                    degree = int(text[:-1])
                    if degree < 0:
                        raise ValueError
                    parity = {"e": 1, "o": -1, "y": (-1) ** degree}[text[-1]]
                except (ValueError, KeyError, IndexError):
                    raise ValueError(f'unable to convert string "{text}" into an Irrep') from None
                l, p = degree, parity
            elif isinstance(l, tuple):
                l, p = l
        if not isinstance(l, int) or l < 0:
            raise ValueError(f"l must be positive integer, got {l}")
        if p not in (-1, 1):
            raise ValueError(f"parity must be on of (-1, 1), got {p}")
        return super().__new__(cls, (l, p))

    @property
    def l(self) -> int:
        return self[0]

    @property
    def p(self) -> int:
        return self[1]

    @property
    def dim(self) -> int:
        return 2 * self.l + 1

    def is_scalar(self) -> bool:
        return self.l == 0 and self.p == 1

    def __repr__(self) -> str:
        return f"{self.l}{'e' if self.p == 1 else 'o'}"

    def __mul__(self, other):
        other = Irrep(other)
        for degree in range(abs(self.l - other.l), self.l + other.l + 1):
            yield Irrep(degree, self.p * other.p)

    def __rmul__(self, other):
        return Irreps([(other, self)])

    def __add__(self, other):
        return Irreps(self) + Irreps(other)


class MulIr(tuple):
    """``mul`` copies of one irrep."""

    def __new__(cls, mul, ir=None):
        if ir is None:
            mul, ir = mul
        if not isinstance(mul, int) or not isinstance(ir, Irrep):
            raise TypeError("MulIr needs an int multiplicity and an Irrep")
        return super().__new__(cls, (mul, ir))

    @property
    def mul(self) -> int:
        return self[0]

    @property
    def ir(self) -> Irrep:
        return self[1]

    @property
    def dim(self) -> int:
        return self.mul * self.ir.dim

    def __repr__(self) -> str:
        return f"{self.mul}x{self.ir}"


class Irreps(tuple):
    """Ordered direct sum of ``MulIr`` blocks, e.g. ``Irreps("32x0e+32x1o")``."""

    def __new__(cls, irreps=None):
        if isinstance(irreps, Irreps):
            return super().__new__(cls, irreps)
        blocks = []
        if isinstance(irreps, Irrep):
            blocks.append(MulIr(1, irreps))
        elif isinstance(irreps, str):
            try:
                for chunk in irreps.split("+") if irreps.strip() else []:
                    if "x" in chunk:
                        mul_text, ir_text = chunk.split("x")
                        mul = int(mul_text)
                    else:
                        mul, ir_text = 1, chunk
                    if mul < 0:
                        raise ValueError
                    blocks.append(MulIr(mul, Irrep(ir_text)))
            except Exception:
                raise ValueError(f'Unable to convert string "{irreps}" into an Irreps') from None
        elif irreps is not None:
            for item in irreps:
                if isinstance(item, (str, Irrep)) and not isinstance(item, MulIr):
                    blocks.append(MulIr(1, Irrep(item)))
                    continue
                mul, ir = item
                if not isinstance(mul, int) or mul < 0:
                    raise ValueError(f'Unable to interpret "{item}" as an irrep.')
                blocks.append(MulIr(mul, Irrep(ir)))
        return super().__new__(cls, blocks)

    @staticmethod
    def spherical_harmonics(lmax: int, p: int = -1) -> "Irreps":
        return Irreps([(1, (l, p ** l)) for l in range(lmax + 1)])

    def slices(self):
        out, start = [], 0
        for block in self:
            out.append(slice(start, start + block.dim))
            start += block.dim
        return out

    def __getitem__(self, index):
        value = super().__getitem__(index)
        return Irreps(value) if isinstance(index, slice) else value

    def __contains__(self, ir) -> bool:
        ir = Irrep(ir)
        return any(block.ir == ir for block in self)

    def count(self, ir) -> int:
        ir = Irrep(ir)
        return sum(block.mul for block in self if block.ir == ir)

    def __add__(self, other) -> "Irreps":
        return Irreps(tuple(self) + tuple(Irreps(other)))

    def __mul__(self, other) -> "Irreps":
        if isinstance(other, Irreps):
            raise NotImplementedError("Use a tensor product for this")
        return Irreps(super().__mul__(other))

    def __rmul__(self, other) -> "Irreps":
        return Irreps(super().__rmul__(other))

    def simplify(self) -> "Irreps":
        out = []
        for mul, ir in self:
            if out and out[-1][1] == ir:
                out[-1] = (out[-1][0] + mul, ir)
            elif mul > 0:
                out.append((mul, ir))
        return Irreps(out)

    def remove_zero_multiplicities(self) -> "Irreps":
        return Irreps([(mul, ir) for mul, ir in self if mul > 0])

    @property
    def dim(self) -> int:
        return sum(block.dim for block in self)

    @property
    def num_irreps(self) -> int:
        return sum(block.mul for block in self)

    @property
    def ls(self) -> list:
        return [ir.l for mul, ir in self for _ in range(mul)]

    @property
    def lmax(self) -> int:
        if len(self) == 0:
            raise ValueError("Cannot get lmax of empty Irreps")
        return max(self.ls)

    def __repr__(self) -> str:
        return "+".join(repr(block) for block in self)


def as_irreps(value: "Irreps | str | Iterable") -> Irreps:
    return value if isinstance(value, Irreps) else Irreps(value)


__all__ = ["Irrep", "Irreps", "MulIr", "as_irreps"]
