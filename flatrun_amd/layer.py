"""The projection chain of one decoder block, activations resident on the GPU.

The reference's decoder block (``_decoder_block``, model/qwen2.py:1388-1773)
calls the backend once per projection with host arrays and glues the
results with NumPy: q, k, v on the normed x and ``np.concatenate``
(:1510-1519), attention, o (:1625-1646), residual and norm, gate and up and
``np.concatenate`` (:1690-1702), SiLU(gate) * up (:1703-1740), down
(:1742-1748). Every call crosses PCIe twice. :class:`DecoderProjections`
keeps every activation of that chain in device buffers:

    x ─▶ [q|k|v] grouped ─▶ qkv ─▶ attention (caller) ─▶ attn
    attn ─▶ o ─▶ o_out ─▶ residual + norm (caller) ─▶ xn
    xn ─▶ [gate|up] grouped ─▶ gateup ─▶ SiLU·mul ─▶ act ─▶ down ─▶ mlp_out

The projections are frq_dev_gemv_group / frq_dev_gemv launches (fp32
contract, 1e-5 of fp64); gate, up and SiLU·mul are frq_dev_gemv_swiglu (one
launch for a Q4_K pair at batch 1, the grouped launch and frq_dev_silu_mul
otherwise, same bits); all on one stream.
Attention, RoPE, norms and residuals are not quantized matvecs; the caller
supplies them as functions on device buffers (or does them itself between
:meth:`qkv`, :meth:`o` and :meth:`mlp`).

o_proj is a projection like the others here. In the reference its native
branch never runs: o's weight comes from ``_fetch_linear_with_quant`` ->
``dequant_handle`` as F32, so the guard ``o_w.dtype != np.float32``
(qwen2.py:1630-1640) is false under the default dtype and o runs as
``attn_out @ o_w.T`` in NumPy even with ``--backend native``; with another
dtype the branch would hand a dequantized array to the kernel as if it
were raw blocks.
"""

from __future__ import annotations

from dataclasses import dataclass

from . import device

PROJECTIONS = ("q", "k", "v", "o", "gate", "up", "down")


@dataclass(frozen=True)
class Projection:
    qtype: str
    weight: object        # DeviceWeight / DeviceBuffer / device address holder (data_ptr())
    n: int                # output features
    k: int                # input features
    nbytes: int


def _proj(spec) -> Projection:
    if isinstance(spec, Projection):
        return spec
    q, w, n, k = spec[:4]
    nb = int(spec[4]) if len(spec) > 4 else int(getattr(w, "nbytes"))
    return Projection(str(q), w, int(n), int(k), nb)


class DecoderProjections:
    """The seven projections of one decoder block on device-resident weights.

    ``weights`` maps "q", "k", "v", "o", "gate", "up", "down" to
    ``(qtype, weight, n, k[, nbytes])`` (or :class:`Projection`): (n, k) =
    (out, in) as in the tensor's metadata shape. Buffers for up to
    ``max_seq`` rows are allocated once: ``qkv`` (q|k|v concatenated per
    row, as the reference concatenates them), ``o_out``, ``gateup``, ``act``
    and ``mlp_out``."""

    def __init__(self, weights: dict, max_seq: int = 1, stream=None):
        missing = [p for p in PROJECTIONS if p not in weights]
        if missing:
            raise ValueError(f"missing projections: {missing}")
        self.p = {name: _proj(weights[name]) for name in PROJECTIONS}
        q, k, v, o, g, u, d = (self.p[n] for n in PROJECTIONS)
        self.hidden = q.k
        if not (k.k == v.k == g.k == u.k == self.hidden):
            raise ValueError("q, k, v, gate and up must share their input size (the hidden size)")
        if g.n != u.n or d.k != g.n:
            raise ValueError("gate and up must have the same outputs, and down take them as input")
        if o.k != q.n:
            raise ValueError("o must take the attention output (q's output size) as input")
        self.inter = g.n
        self.qkv_n = q.n + k.n + v.n
        self.max_seq = int(max_seq)
        if self.max_seq < 1:
            raise ValueError("max_seq must be >= 1")
        self.stream = stream
        s = self.max_seq
        self.qkv = device.DeviceBuffer(4 * s * self.qkv_n)
        self.o_out = device.DeviceBuffer(4 * s * o.n)
        self.gateup = device.DeviceBuffer(4 * s * 2 * self.inter)
        self.act = device.DeviceBuffer(4 * s * self.inter)
        self.mlp_out = device.DeviceBuffer(4 * s * d.n)

    def _check_seq(self, seq: int) -> int:
        seq = int(seq)
        if not 1 <= seq <= self.max_seq:
            raise ValueError(f"seq must be in 1..{self.max_seq}, got {seq}")
        return seq

    def _gemv(self, name: str, x, y, seq: int) -> None:
        p = self.p[name]
        device.gemv(p.qtype, p.weight, x, y, p.n, p.k, batch=seq, stream=self.stream, w_bytes=p.nbytes)

    def qkv_proj(self, x, seq: int = 1):
        """qkv[r] = [W_q x_r | W_k x_r | W_v x_r] (x: seq rows of hidden floats
        on the device); returns the qkv buffer."""
        seq = self._check_seq(seq)
        q, k, v = self.p["q"], self.p["k"], self.p["v"]
        base = self.qkv.ptr
        device.gemv_group([(q.qtype, q.weight, q.n, base, q.nbytes),
                           (k.qtype, k.weight, k.n, base + 4 * q.n, k.nbytes),
                           (v.qtype, v.weight, v.n, base + 4 * (q.n + k.n), v.nbytes)],
                          x, self.hidden, batch=seq, y_stride=self.qkv_n, stream=self.stream)
        return self.qkv

    def o_proj(self, attn, seq: int = 1):
        """o_out = W_o attn (attn: seq rows of q.n floats); returns o_out."""
        seq = self._check_seq(seq)
        self._gemv("o", attn, self.o_out, seq)
        return self.o_out

    def mlp(self, xn, seq: int = 1):
        """mlp_out = W_down (silu(W_gate xn) * W_up xn); returns mlp_out."""
        seq = self._check_seq(seq)
        g, u = self.p["gate"], self.p["up"]
        device.gemv_swiglu((g.qtype, g.weight, g.n, g.nbytes), (u.qtype, u.weight, u.n, u.nbytes), xn,
                           self.hidden, self.gateup, self.act, batch=seq, stream=self.stream)
        self._gemv("down", self.act, self.mlp_out, seq)
        return self.mlp_out

    def forward(self, x, seq: int = 1, attention=None, post_attention=None):
        """The chain with the caller's non-matvec steps between:
        ``attention(qkv, seq) -> attn`` (device buffer of seq x q.n floats)
        and ``post_attention(o_out, seq) -> xn`` (seq x hidden; residual and
        norm). Returns mlp_out (the block's MLP output before its residual).
        Enqueued on the stream; synchronise before reading."""
        if attention is None or post_attention is None:
            raise ValueError("forward needs the attention and post_attention steps")
        attn = attention(self.qkv_proj(x, seq), seq)
        xn = post_attention(self.o_proj(attn, seq), seq)
        return self.mlp(xn, seq)

    def close(self) -> None:
        for b in (self.qkv, self.o_out, self.gateup, self.act, self.mlp_out):
            b.free()

    def __enter__(self) -> "DecoderProjections":
        return self

    def __exit__(self, *exc) -> None:
        self.close()
