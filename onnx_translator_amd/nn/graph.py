"""Graph executor (``nn/__init__.py:346-505`` of the reference), device-resident.

Same constructor and naming as the reference ``Graph``; the differences fix its
gaps and keep the data in HBM:

* initializers are fed (the reference never feeds them, ``nn/__init__.py:423-424``);
  ``to_device()`` uploads them once, so weights stay resident across calls;
* ``forward`` returns the graph outputs (the reference returns nothing);
* graph inputs are moved to the device once and every intermediate stays there
  (each operator with a device operand writes a device tensor); an edge is
  released when its last consumer has run;
* ``fuse_elementwise()`` replaces runs of consecutive float32 Relu / Abs / Cos /
  Add / Sub / Mul / Div nodes whose intermediates have no other consumer by one
  :class:`~onnx_translator_amd.nn.Operators.ElementwiseChain` (bit-identical to
  the unfused run).  Shapes are taken from a placeholder pass (``forward_``) at
  the first call, when the input shapes are known;
* ``fuse()`` also replaces a DequantizeLinear of int8 / uint8 codes whose only
  consumer is a Gemm's B input by one
  :class:`~onnx_translator_amd.nn.Operators.DequantizeGemm` (the
  weight-only-quantized Gemm reads the codes; bit-identical to the pair);
* ``fuse()`` also folds a Conv whose output feeds only a Relu, and that
  Relu's (or the Conv's) output feeds only an Add with an operand of the same
  shape, into one :class:`~onnx_translator_amd.nn.Operators.FusedConv`
  (``conv2d_fused_forward``; bit-identical to the sequence), placed where the
  last folded node was; and evaluates DequantizeLinear nodes whose inputs are
  all initializers once (their outputs become initializers).  On request
  (``fuse(dequantize_conv=True)``) it also folds a per-tensor DequantizeLinear
  of uint8 / int8 codes whose consumers are all convolutions into each of them
  (:class:`~onnx_translator_amd.nn.Operators.DequantizeConv`, which reads the
  codes: 4x smaller activations, but on MI355X the byte gather costs more than
  the separate DequantizeLinear pass it saves, so it is off by default);
* a missing QuantizeLinear / DequantizeLinear zero point is a uint8 zero (the
  ONNX default).
"""
from __future__ import annotations

import sys
from collections import OrderedDict
from typing import Dict, List, Optional

import numpy as np

from . import NUMPY_TO_DTYPE, Tensor, Tensor_
from . import Operators as Op

_UNARY = {Op.RELU: "Relu", Op.ABS: "Abs", Op.COS: "Cos"}
_BINARY = {Op.ADD: "Add", Op.SUB: "Sub", Op.MUL: "Mul", Op.DIV: "Div"}


def _is_fusable(op) -> bool:
    return type(op) in _UNARY or type(op) in _BINARY


class Graph:
    """Operators in topological order over named edges."""

    def __init__(self, ops, input_name, output_name=None, model_name=None,
                 initializers: Optional[Dict[str, Tensor]] = None):
        self.input_name = list(input_name) if isinstance(input_name, (list, tuple)) else [input_name]
        if output_name is None:
            self.output_name: List[str] = []
        else:
            self.output_name = list(output_name) if isinstance(output_name, (list, tuple)) else [output_name]
        self.model_name = model_name
        self.initializers: Dict[str, Tensor] = dict(initializers or {})
        self.ops: "OrderedDict[str, object]" = OrderedDict()
        self._fuse_pending = None      # passes requested by fuse(), applied at the first forward
        self.device = False
        self.fused_runs: List[List[str]] = []
        self.folded: List[str] = []
        self.update(ops)

    # -- structure ---------------------------------------------------------------
    def update(self, ops):
        """Name the operators (``<Class>.<k>``) and check single assignment of edges."""
        counts: Dict[str, int] = {}
        produced = set(self.input_name) | set(self.initializers)
        for op in ops:
            cls = type(op).__name__
            counts[cls] = counts.get(cls, -1) + 1
            if not getattr(op, "name", None):
                op.name = f"{cls}.{counts[cls]}"
            self.ops[op.name] = op
            for o in op.outputs:
                if o in produced and o not in self.initializers:
                    print(f"output edge name {o} repeat!!!")
                    sys.exit()
                produced.add(o)
        if not self.output_name:
            consumed = {i for op in self.ops.values() for i in op.inputs}
            self.output_name = [o for op in self.ops.values() for o in op.outputs if o not in consumed]

    def _consumers(self) -> Dict[str, int]:
        c: Dict[str, int] = {}
        for op in self.ops.values():
            for i in op.inputs:
                if i:
                    c[i] = c.get(i, 0) + 1
        for o in self.output_name:
            c[o] = c.get(o, 0) + 1
        return c

    def to_device(self) -> "Graph":
        """Upload the initializers to HBM once; inputs given to ``forward`` go to HBM too."""
        self.initializers = {k: (v.to_device() if isinstance(v, Tensor) else v) for k, v in self.initializers.items()}
        self.device = True
        return self

    # -- execution ----------------------------------------------------------------
    @staticmethod
    def _inputs_for(op, buf):
        args = [buf[na] if na else None for na in op.inputs]
        if type(op) in (Op.QuantizeLinear, Op.DequantizeLinear) and len(args) == 2:
            args.append(Tensor(1, dtype="uint8", data=np.zeros(1, np.uint8)))
        return args

    def _run(self, inputs, method: str):
        # Shape propagation also sees the initializers themselves: they carry size
        # and dtype like a placeholder, and operators whose output shape depends
        # on a value (Reshape's shape input) read it.
        buf: Dict[str, object] = dict(self.initializers)
        for na, t in zip(self.input_name, inputs):
            buf[na] = t
        pending = self._consumers()
        for op in self.ops.values():
            outs = getattr(op, method)(*self._inputs_for(op, buf))
            res = outs["tensor"]
            if len(op.outputs) == 1:
                buf[op.outputs[0]] = res
            else:
                for na, r in zip(op.outputs, res):
                    buf[na] = r
            for na in op.inputs:
                if not na or na in self.initializers:
                    continue
                pending[na] -= 1
                if pending[na] == 0:
                    buf.pop(na, None)
        out = tuple(buf[na] for na in self.output_name)
        return out[0] if len(out) == 1 else out

    def forward(self, *inputs):
        """Run the graph; inputs may be numpy arrays or :class:`Tensor` objects.  Host
        inputs are moved to the device after ``to_device()``.  Returns the output
        tensor(s) (device-resident when computed there; ``.numpy()`` copies back)."""
        ts = []
        dev = self.device
        for x in inputs:
            if not isinstance(x, Tensor):
                a = np.ascontiguousarray(x)
                x = Tensor(*a.shape, dtype=NUMPY_TO_DTYPE.get(a.dtype.type, "float32"), data=a)
            ts.append(x.to_device() if dev and not x.on_device else x)
        if self._fuse_pending is not None:
            self._fuse(ts)
        return self._run(ts, "forward")

    def forward_(self, *inputs):
        """Shape / dtype propagation with :class:`Tensor_` placeholders."""
        return self._run(inputs, "forward_")

    # -- fusion --------------------------------------------------------------------
    def fuse(self, elementwise: bool = True, dequantize_gemm: bool = True, conv_epilogue: bool = True,
             fold_constants: bool = True, dequantize_conv: bool = False,
             quantize_dequantize: bool = True, pool_quantize_dequantize: bool = False,
             int8_conv: bool = False, gemm_softmax: bool = True) -> "Graph":
        """Request the graph passes; they are applied at the first ``forward`` (shapes needed).
        ``dequantize_conv`` folds activation DequantizeLinear nodes into their convolutions
        and so takes precedence over ``quantize_dequantize`` for those pairs.
        ``pool_quantize_dequantize`` lets a MaxPool write the fake-quantized copy of its
        output as well (MaxPoolQDQ); off by default, as on the config-5 graph the pooling
        kernel with two outputs is slower than the two separate passes.
        ``int8_conv`` (device graphs) runs QDQ residual blocks on the int8 MFMA kernels
        (QuantizeNHWC, QConvBlock): their convolutions sum the integer codes exactly and
        scale once, the tolerance class of the MFMA convolution rather than the bits of the
        operator sequence, and they have no exact mode, so it is off by default.
        ``gemm_softmax`` (device graphs) runs a Gemm whose f32 output only a Softmax over
        its last axis reads as one GemmSoftmax (bit for bit; the Gemm's split reduction
        takes the softmax)."""
        self._fuse_pending = (elementwise, dequantize_gemm, conv_epilogue, fold_constants, dequantize_conv,
                              quantize_dequantize, pool_quantize_dequantize, int8_conv, gemm_softmax)
        return self

    def fuse_elementwise(self) -> "Graph":
        """Request elementwise fusion only."""
        return self.fuse(True, False, False, False, False, False, False, False, False)

    def _edge_shapes(self, inputs) -> Dict[str, tuple]:
        shapes: Dict[str, tuple] = {k: (tuple(v.size), v.dtype) for k, v in self.initializers.items()}
        buf: Dict[str, object] = dict(self.initializers)     # value-dependent shapes (Reshape) read them
        for na, t in zip(self.input_name, inputs):
            buf[na] = Tensor_(*t.size, dtype=t.dtype)
            shapes[na] = (tuple(t.size), t.dtype)
        for op in self.ops.values():
            res = op.forward_(*self._inputs_for(op, buf))["tensor"]
            res = [res] if len(op.outputs) == 1 else list(res)
            for na, r in zip(op.outputs, res):
                buf[na] = r
                shapes[na] = (tuple(r.size), r.dtype)
        return shapes

    def _fuse(self, inputs):
        elementwise, dq_gemm, conv_epi, fold, dq_conv, qdq, pool_qdq, int8_conv, gemm_sm = self._fuse_pending
        self._fuse_pending = None
        shapes = self._edge_shapes(inputs)
        if int8_conv and self.device and self._fuse_qconv_blocks(shapes, self._consumers()):
            shapes = self._edge_shapes(inputs)
        if dq_gemm:
            self._fuse_dq_gemm(shapes, self._consumers())
        if fold:
            self._fold_constants()
        if conv_epi:
            self._fuse_conv_epilogue(shapes, self._consumers())
        if dq_conv:
            self._fuse_dq_conv(shapes)
        if qdq:
            self._fuse_qdq(shapes, self._consumers())
            if conv_epi:
                self._fuse_conv_qdq(shapes, self._consumers())
            if pool_qdq:
                self._fuse_pool_qdq(shapes)
        if gemm_sm and self.device:
            self._fuse_gemm_softmax(shapes)
        if elementwise:
            self._fuse_gap_flatten(shapes, self._consumers())
            self._fuse_runs(shapes, self._consumers())

    def _fuse_gemm_softmax(self, shapes):
        """A float32 Gemm whose output is read only by a Softmax over its last axis
        becomes one GemmSoftmax with both outputs (the Gemm's output stays an edge)."""
        ops = list(self.ops.values())
        users: Dict[str, list] = {}
        for op in ops:
            for na in op.inputs:
                if na:
                    users.setdefault(na, []).append(op)
        replace, drop = {}, set()
        for op in ops:
            if type(op) is not Op.Gemm or op.dtype != "float32":
                continue
            y = op.outputs[0]
            u = users.get(y, [])
            if len(u) != 1 or type(u[0]) is not Op.Softmax or y not in shapes or shapes[y][1] != "float32":
                continue
            sm = u[0]
            nd = len(shapes[y][0])
            if sm.dtype not in (None, "float32") or sm.axis not in (nd - 1, -1):
                continue
            fused = Op.GemmSoftmax(list(op.inputs), [y, sm.outputs[0]], op.alpha, op.beta, op.transA, op.transB,
                                   op.dtype)
            fused.name = f"GemmSoftmax.{op.name}+{sm.name}"
            replace[op.name] = fused
            drop.add(sm.name)
            self.fused_runs.append([op.name, sm.name])
        if replace:
            self.ops = OrderedDict((o.name, o) for o in [replace.get(o.name, o) for o in ops if o.name not in drop])

    def _fuse_qconv_blocks(self, shapes, consumers) -> bool:
        """QDQ residual blocks onto the int8 MFMA kernels.  A block is
        QuantizeLinear -> DequantizeLinear (one-element uint8 / int8 parameters) ->
        Conv (group 1, dilation 1) whose weight is a DequantizeLinear of int8
        codes along axis 0 with zero points 0, [-> Relu] [-> Add with a tensor of
        the output's shape, or with a 1x1 / pads-0 Conv of the same activation and
        strides, no bias, whose weight is such a DequantizeLinear], with C % 32 ==
        0 and M % 64 == 0, and nothing else reading its intermediates.  It becomes
        one QConvBlock at its last node; its input codes come from a QuantizeNHWC
        at the QuantizeLinear's place, or straight from the previous block when
        that block's output is read only by this block's QuantizeLinear.  The
        weights are repacked once, channels-last with per-tap code sums, as new
        device initializers.  Returns whether anything was replaced."""
        ops = list(self.ops.values())
        producer = {o: op for op in ops for o in op.outputs}
        users: Dict[str, list] = {}
        for op in ops:
            for na in op.inputs:
                if na:
                    users.setdefault(na, []).append(op)
        init = self.initializers

        def only(edge):
            u = users.get(edge, [])
            return u[0] if len(u) == 1 and consumers.get(edge, 0) == 1 and edge not in self.output_name else None

        def one(edge, dt):
            return bool(edge) and edge in init and shapes[edge][1] == dt and int(np.prod(shapes[edge][0] or (1,))) == 1

        def weight(edge, conv):
            """(dq node, int8 codes, scales [M]) of a weight read only by conv, or None."""
            dq = producer.get(edge)
            if type(dq) is not Op.DequantizeLinear or only(edge) is not conv or dq.axis not in (0, -4):
                return None
            q, sc = dq.inputs[0], dq.inputs[1]
            z = dq.inputs[2] if len(dq.inputs) > 2 else ""
            if q not in init or sc not in init or (z and z not in init) or shapes[q][1] != "int8":
                return None
            if len(shapes[q][0]) != 4 or shapes[sc][1] != "float32":
                return None
            m = shapes[q][0][0]
            sv = init[sc].numpy().reshape(-1)
            if sv.size != m or (z and np.any(init[z].numpy() != 0)):
                return None
            return dq, init[q].numpy(), sv.astype(np.float32)

        blocks = []
        for c in ops:
            if type(c) is not Op.Conv or c.group != 1 or c.dtype not in (None, "float32") or tuple(c.dilations) != (1, 1):
                continue
            xd = c.inputs[0]
            dqx = producer.get(xd)
            if type(dqx) is not Op.DequantizeLinear or len(dqx.inputs) < 2:
                continue
            xq = dqx.inputs[0]
            qx = producer.get(xq)
            if type(qx) is not Op.QuantizeLinear or only(xq) is not dqx or len(qx.inputs) < 2:
                continue
            cdt = shapes[xq][1]
            qs, qz = qx.inputs[1], (qx.inputs[2] if len(qx.inputs) > 2 else "")
            ds, dz = dqx.inputs[1], (dqx.inputs[2] if len(dqx.inputs) > 2 else "")
            if cdt not in ("uint8", "int8") or not one(qs, "float32") or not one(ds, "float32"):
                continue
            if (qz and not one(qz, cdt)) or (dz and not one(dz, cdt)):
                continue
            xs = shapes[qx.inputs[0]]
            if xs[1] != "float32" or len(xs[0]) != 4 or xs[0][1] % 32:
                continue
            wt = weight(c.inputs[1], c)
            if wt is None or wt[1].shape[0] % 64 or wt[1].shape[1] != xs[0][1]:
                continue
            b = c.inputs[2] if len(c.inputs) > 2 else ""
            if b and (b not in init or shapes[b][1] != "float32" or int(np.prod(shapes[b][0])) != wt[1].shape[0]):
                continue
            chain, cur, relu, skip, proj, pw = [c], c.outputs[0], False, "", None, None
            nxt = only(cur)
            if type(nxt) is Op.RELU and nxt.dtype in (None, "float32"):
                chain.append(nxt)
                cur, relu = nxt.outputs[0], True
                nxt = only(cur)
            if (type(nxt) is Op.ADD and nxt.dtype in (None, "float32") and len(nxt.inputs) == 2 and
                    nxt.inputs.count(cur) == 1 and shapes[nxt.outputs[0]][0] == shapes[cur][0]):
                other = nxt.inputs[1 - nxt.inputs.index(cur)]
                po = producer.get(other)
                if (type(po) is Op.Conv and po is not c and po.inputs[0] == xd and only(other) is nxt and
                        po.group == 1 and tuple(po.dilations) == (1, 1) and tuple(po.pads) == (0, 0, 0, 0) and
                        tuple(po.strides) == tuple(c.strides) and (len(po.inputs) < 3 or not po.inputs[2]) and
                        shapes[other][0] == shapes[cur][0]):
                    pw = weight(po.inputs[1], po)
                    if pw is not None and pw[1].shape[2:] == (1, 1):
                        proj = po
                if proj is None and shapes[other][1] == "float32" and shapes[other][0] == shapes[cur][0]:
                    skip = other
                if proj is not None or skip:
                    chain.append(nxt)
                    cur = nxt.outputs[0]
            # the activation must feed this block only
            if set(o.name for o in users.get(xd, [])) != {c.name} | ({proj.name} if proj else set()):
                continue
            if proj is not None:
                chain.insert(1, proj)
            blocks.append(dict(c=c, qx=qx, dqx=dqx, xq=xq, cdt=cdt, qs=qs, qz=qz, ds=ds, dz=dz, w=wt, b=b,
                               relu=relu, skip=skip, proj=proj, pw=pw, chain=chain, out=cur, src=None, nxt=None))
        if not blocks:
            return False
        by_qx = {bl["qx"].name: bl for bl in blocks}
        for bl in blocks:
            u = only(bl["out"])
            if type(u) is Op.QuantizeLinear and u.name in by_qx:
                bl["nxt"] = by_qx[u.name]
                by_qx[u.name]["src"] = bl

        def put(name, arr, dt):
            t = Tensor(*arr.shape, dtype=dt, data=np.ascontiguousarray(arr)).to_device()
            self.initializers[name] = t
            return name

        def packed(prefix, codes, scales):
            k = codes.transpose(0, 2, 3, 1)
            return (put(prefix + ".qk", k, "int8"), put(prefix + ".qsum", k.sum(axis=3, dtype=np.int64).astype(np.int32),
                                                        "int32"), put(prefix + ".qscale", scales, "float32"))

        replace, drop = {}, set()
        for bl in blocks:
            c = bl["c"]
            codes_in = bl["xq"] + ".nhwc"
            if bl["src"] is None:
                x = bl["qx"].inputs[0]
                mp = producer.get(x)
                if (type(mp) is Op.MaxPool and mp.dtype == "float32" and shapes[x][1] == "float32" and
                        list(mp.kernel_shape) == [3, 3] and list(mp.strides) == [2, 2] and
                        list(mp.pads)[:2] == [1, 1] and list(mp.dilations) == [1, 1] and mp.name not in replace):
                    # the MaxPool writes the codes as well: its output is read once
                    qn = Op.MaxPoolQuantizeNHWC([mp.inputs[0], bl["qs"], bl["qz"]], [x, codes_in], mp.kernel_shape,
                                                mp.pads, mp.strides, mp.dtype, bl["cdt"], mp.dilations)
                    qn.name = f"MaxPoolQuantizeNHWC.{mp.name}+{bl['qx'].name}"
                    replace[mp.name] = qn
                    drop.add(bl["qx"].name)
                else:
                    qn = Op.QuantizeNHWC([x, bl["qs"], bl["qz"]], [codes_in], bl["cdt"])
                    qn.name = f"QuantizeNHWC.{bl['qx'].name}"
                    replace[bl["qx"].name] = qn
            else:
                drop.add(bl["qx"].name)
            wk, wsum, wsc = packed(c.name, bl["w"][1], bl["w"][2])
            pk = psum = psc = ""
            if bl["proj"] is not None:
                pk, psum, psc = packed(bl["proj"].name, bl["pw"][1], bl["pw"][2])
            nb = bl["nxt"]
            out = nb["xq"] + ".nhwc" if nb else bl["out"]
            blk = Op.QConvBlock([codes_in, bl["ds"], bl["dz"], wk, wsum, wsc, bl["b"], pk, psum, psc, bl["skip"],
                                 nb["qs"] if nb else "", nb["qz"] if nb else ""], [out], c.pads, c.strides,
                                c.dilations, bl["relu"], bl["cdt"], nb["cdt"] if nb else None)
            blk.name = "QConvBlock." + "+".join(o.name for o in bl["chain"])
            replace[bl["chain"][-1].name] = blk
            drop.update(o.name for o in bl["chain"][:-1])
            drop.update({bl["dqx"].name, bl["w"][0].name} | ({bl["pw"][0].name} if bl["proj"] is not None else set()))
            self.fused_runs.append([bl["qx"].name, bl["dqx"].name] + [o.name for o in bl["chain"]])
        out = [replace.get(o.name, o) for o in ops if o.name not in drop]
        self.ops = OrderedDict((o.name, o) for o in out)
        return True

    def _fold_constants(self):
        """DequantizeLinear nodes over initializers only are evaluated once."""
        out = []
        for op in self.ops.values():
            ins = [na for na in op.inputs if na]
            if type(op) is Op.DequantizeLinear and ins and all(na in self.initializers for na in ins):
                args = self._inputs_for(op, self.initializers)
                self.initializers[op.outputs[0]] = op.forward(*args)["tensor"]
                self.folded.append(op.name)
                continue
            out.append(op)
        self.ops = OrderedDict((o.name, o) for o in out)

    def _fuse_conv_epilogue(self, shapes, consumers):
        ops = list(self.ops.values())
        users: Dict[str, list] = {}
        for op in ops:
            for na in op.inputs:
                if na:
                    users.setdefault(na, []).append(op)

        def only_user(edge):
            u = users.get(edge, [])
            return u[0] if len(u) == 1 and consumers.get(edge, 0) == 1 and edge not in self.output_name else None

        def f32(edge):
            return edge in shapes and shapes[edge][1] == "float32"

        replace, drop = {}, set()
        for op in ops:
            if type(op) is not Op.Conv or op.dtype != "float32" or not f32(op.outputs[0]):
                continue
            chain, cur, relu, skip = [op], op.outputs[0], False, ""
            nxt = only_user(cur)
            if type(nxt) is Op.RELU and f32(nxt.outputs[0]) and nxt.dtype in (None, "float32"):
                chain.append(nxt)
                cur, relu = nxt.outputs[0], True
                nxt = only_user(cur)
            if (type(nxt) is Op.ADD and nxt.dtype in (None, "float32") and len(nxt.inputs) == 2 and
                    nxt.inputs.count(cur) == 1):
                other = nxt.inputs[1 - nxt.inputs.index(cur)]
                if f32(other) and shapes[other][0] == shapes[cur][0] == shapes[nxt.outputs[0]][0]:
                    chain.append(nxt)
                    cur, skip = nxt.outputs[0], other
            if len(chain) == 1 or any(o.name in drop or o.name in replace for o in chain):
                continue
            b = op.inputs[2] if len(op.inputs) > 2 else ""
            fc = Op.FusedConv([op.inputs[0], op.inputs[1], b, skip], [cur], op.pads, op.strides, op.dilations,
                              op.group, op.dtype, relu)
            fc.name = "FusedConv." + "+".join(o.name for o in chain)
            replace[chain[-1].name] = fc
            drop.update(o.name for o in chain[:-1])
            self.fused_runs.append([o.name for o in chain])
        out = [replace.get(o.name, o) for o in ops if o.name not in drop]
        self.ops = OrderedDict((o.name, o) for o in out)

    @staticmethod
    def _dq_axis(dq, shapes):
        """Axis of a DequantizeLinear's parameters over its 2-D input as
        ``DequantizeLinear.forward`` applies them, or None if they are not
        per-tensor / per-row / per-column."""
        xs = shapes[dq.inputs[0]][0]
        ss = shapes[dq.inputs[1]][0]
        size = int(np.prod(ss)) if ss else 1
        if size == 1:
            return 0
        if len(ss) == 1:
            axis = dq.axis if dq.axis is not None else 1     # numpy broadcasting aligns with the last dim
            axis = axis + 2 if axis < 0 else axis
            return axis if axis in (0, 1) and xs[axis] == ss[0] else None
        if tuple(ss) == (xs[0], 1):
            return 0
        if tuple(ss) in ((1, xs[1]),):
            return 1
        return None

    def _fuse_dq_gemm(self, shapes, consumers):
        ops = list(self.ops.values())
        producer = {o: op for op in ops for o in op.outputs}
        out, drop = [], set()
        for op in ops:
            fused = None
            if type(op) is Op.Gemm and len(op.inputs) >= 2 and op.inputs[1]:
                b = op.inputs[1]
                dq = producer.get(b)
                ok = (type(dq) is Op.DequantizeLinear and consumers.get(b, 0) == 1 and
                      b not in self.output_name and b not in op.inputs[:1] + op.inputs[2:] and
                      shapes.get(dq.inputs[0], ((), ""))[1] in ("int8", "uint8") and
                      len(shapes[dq.inputs[0]][0]) == 2 and shapes[b][1] == "float32")
                zp_ok = ok and (len(dq.inputs) < 3 or not dq.inputs[2] or (
                    int(np.prod(shapes[dq.inputs[2]][0] or (1,))) == int(np.prod(shapes[dq.inputs[1]][0] or (1,))) or
                    int(np.prod(shapes[dq.inputs[2]][0] or (1,))) == 1))
                axis = self._dq_axis(dq, shapes) if zp_ok else None
                if axis is not None:
                    zp = dq.inputs[2] if len(dq.inputs) > 2 else ""
                    fused = Op.DequantizeGemm([op.inputs[0], dq.inputs[0], dq.inputs[1], zp] + list(op.inputs[2:3]),
                                              list(op.outputs), op.alpha, op.beta, op.transA, op.transB, axis,
                                              op.dtype)
                    fused.name = f"DequantizeGemm.{dq.name}+{op.name}"
                    drop.add(dq.name)
                    self.fused_runs.append([dq.name, op.name])
            out.append(fused or op)
        self.ops = OrderedDict((o.name, o) for o in out if o.name not in drop)

    def _fuse_qdq(self, shapes, consumers):
        """QuantizeLinear -> DequantizeLinear with one-element f32 scales and
        zero points of the code dtype, the codes read by that DequantizeLinear
        only: one QuantizeDequantize at the DequantizeLinear's place (the codes
        are never written)."""
        ops = list(self.ops.values())
        producer = {o: op for op in ops for o in op.outputs}

        def one(edge, dt):
            return bool(edge) and edge in shapes and int(np.prod(shapes[edge][0] or (1,))) == 1 and shapes[edge][1] == dt

        replace, drop = {}, set()
        for dq in ops:
            if type(dq) is not Op.DequantizeLinear or len(dq.inputs) < 3 or not dq.outputs[0]:
                continue
            codes = dq.inputs[0]
            q = producer.get(codes)
            if type(q) is not Op.QuantizeLinear or len(q.inputs) < 3 or q.name in drop:
                continue
            if consumers.get(codes, 0) != 1 or codes in self.output_name or codes in dq.inputs[1:]:
                continue
            cdt = shapes.get(codes, ((), ""))[1]
            if cdt not in ("uint8", "int8", "float8_e4m3", "float8_e5m2"):
                continue
            x, qs, qz = q.inputs[:3]
            ds, dz = dq.inputs[1:3]
            if not (one(qs, "float32") and one(qz, cdt) and one(ds, "float32") and one(dz, cdt)):
                continue
            if shapes.get(x, ((), ""))[1] != "float32" or shapes[dq.outputs[0]][1] != "float32":
                continue
            fused = Op.QuantizeDequantize([x, qs, qz, ds, dz], list(dq.outputs), cdt)
            fused.name = f"QuantizeDequantize.{q.name}+{dq.name}"
            replace[dq.name] = fused
            drop.add(q.name)
            self.fused_runs.append([q.name, dq.name])
        out = [replace.get(o.name, o) for o in ops if o.name not in drop]
        self.ops = OrderedDict((o.name, o) for o in out)

    def _ready_before(self, ops, name, edges) -> bool:
        """True when every edge is a graph input, an initializer, or an output of an
        operator placed before ``name`` in ``ops`` (so a fused operator put at
        ``name``'s position can read it)."""
        before = set(self.input_name) | set(self.initializers)
        for op in ops:
            if op.name == name:
                break
            before.update(op.outputs)
        return all(not e or e in before for e in edges)

    def _fuse_conv_qdq(self, shapes, consumers):
        """Conv / FusedConv (f32) whose output is read only by a QuantizeDequantize
        with uint8 / int8 codes: one FusedConvQDQ in the convolution's place that
        writes the QuantizeDequantize's output (the pre-quantization tensor is
        never written)."""
        ops = list(self.ops.values())
        producer = {o: op for op in ops for o in op.outputs}
        replace, drop = {}, set()
        for fq in ops:
            if type(fq) is not Op.QuantizeDequantize or fq.code_dtype not in ("uint8", "int8"):
                continue
            x = fq.inputs[0]
            c = producer.get(x)
            if type(c) not in (Op.Conv, Op.FusedConv) or c.dtype != "float32" or c.name in replace:
                continue
            if consumers.get(x, 0) != 1 or x in self.output_name or x in fq.inputs[1:]:
                continue
            if not self._ready_before(ops, c.name, fq.inputs[1:5]):
                continue                       # a scale / zero point is produced after the conv
            b = c.inputs[2] if len(c.inputs) > 2 else ""
            skip = c.inputs[3] if type(c) is Op.FusedConv and len(c.inputs) > 3 else ""
            relu = c.relu if type(c) is Op.FusedConv else 0
            fused = Op.FusedConvQDQ([c.inputs[0], c.inputs[1], b, skip] + list(fq.inputs[1:5]), list(fq.outputs),
                                    c.pads, c.strides, c.dilations, c.group, c.dtype, relu, fq.code_dtype)
            fused.name = f"FusedConvQDQ.{c.name}+{fq.name}"
            replace[c.name] = fused
            drop.add(fq.name)
            self.fused_runs.append([c.name, fq.name])
        out = [replace.get(o.name, o) for o in ops if o.name not in drop]
        self.ops = OrderedDict((o.name, o) for o in out)

    def _fuse_gap_flatten(self, shapes, consumers):
        """GlobalAveragePool -> Flatten(axis 1) with the pooled [N, C, 1, 1] tensor
        read by the Flatten only: the pool writes the [N, C] output itself (same
        bytes), and the Flatten's copy goes."""
        ops = list(self.ops.values())
        producer = {o: op for op in ops for o in op.outputs}
        replace, drop = {}, set()
        for fl in ops:
            if type(fl) is not Op.Flatten or fl.axis not in (1, -3):
                continue
            x = fl.inputs[0]
            gp = producer.get(x)
            if type(gp) is not Op.GlobalAveragePool or gp.flatten or gp.name in replace:
                continue
            if consumers.get(x, 0) != 1 or x in self.output_name or len(shapes.get(x, ((),))[0]) != 4:
                continue
            if shapes[x][1] != shapes[fl.outputs[0]][1]:
                continue
            fused = Op.GlobalAveragePool(list(gp.inputs), list(fl.outputs), gp.dtype, gp.version, flatten=True)
            fused.name = f"GlobalAveragePool.{gp.name}+{fl.name}"
            replace[gp.name] = fused
            drop.add(fl.name)
            self.fused_runs.append([gp.name, fl.name])
        out = [replace.get(o.name, o) for o in ops if o.name not in drop]
        self.ops = OrderedDict((o.name, o) for o in out)

    def _fuse_pool_qdq(self, shapes):
        """MaxPool (f32) whose output a QuantizeDequantize with uint8 / int8 codes
        reads: one MaxPoolQDQ in the MaxPool's place with both outputs (the pooled
        tensor keeps its other readers, e.g. a residual Add), so the pooled
        tensor is not read back for the fake quantization."""
        ops = list(self.ops.values())
        producer = {o: op for op in ops for o in op.outputs}
        replace, drop = {}, set()
        for fq in ops:
            if type(fq) is not Op.QuantizeDequantize or fq.code_dtype not in ("uint8", "int8"):
                continue
            x = fq.inputs[0]
            mp = producer.get(x)
            if type(mp) is not Op.MaxPool or mp.dtype != "float32" or mp.name in replace or x in fq.inputs[1:]:
                continue
            if not self._ready_before(ops, mp.name, fq.inputs[1:5]):
                continue                       # a scale / zero point is produced after the pool
            fused = Op.MaxPoolQDQ([mp.inputs[0]] + list(fq.inputs[1:5]), [x, fq.outputs[0]], mp.kernel_shape,
                                  mp.pads, mp.strides, mp.dtype, fq.code_dtype, mp.dilations)
            fused.name = f"MaxPoolQDQ.{mp.name}+{fq.name}"
            replace[mp.name] = fused
            drop.add(fq.name)
            self.fused_runs.append([mp.name, fq.name])
        out = [replace.get(o.name, o) for o in ops if o.name not in drop]
        self.ops = OrderedDict((o.name, o) for o in out)

    def _fuse_dq_conv(self, shapes):
        """DequantizeLinear (per-tensor, uint8 / int8 codes) -> every consuming
        Conv / FusedConv becomes a DequantizeConv; the DequantizeLinear goes."""
        ops = list(self.ops.values())
        users: Dict[str, list] = {}
        for op in ops:
            for na in op.inputs:
                if na:
                    users.setdefault(na, []).append(op)

        def one(edge):
            return edge and edge in shapes and int(np.prod(shapes[edge][0] or (1,))) == 1

        replace, drop = {}, set()
        for dq in ops:
            if type(dq) is not Op.DequantizeLinear or not dq.outputs[0] or dq.outputs[0] in self.output_name:
                continue
            xe, out = dq.inputs[0], dq.outputs[0]
            code_dt = shapes.get(xe, ((), ""))[1]
            zp = dq.inputs[2] if len(dq.inputs) > 2 else ""
            if code_dt not in ("uint8", "int8") or not one(dq.inputs[1]) or shapes[dq.inputs[1]][1] != "float32":
                continue
            if zp and (not one(zp) or shapes[zp][1] != code_dt):
                continue
            cons = users.get(out, [])
            if not cons or any(type(c) not in (Op.Conv, Op.FusedConv) or c.inputs[0] != out or
                               out in c.inputs[1:] or c.dtype != "float32" for c in cons):
                continue
            for c in cons:
                b = c.inputs[2] if len(c.inputs) > 2 else ""
                skip = c.inputs[3] if type(c) is Op.FusedConv else ""
                relu = c.relu if type(c) is Op.FusedConv else 0
                dc = Op.DequantizeConv([xe, dq.inputs[1], zp, c.inputs[1], b, skip], list(c.outputs), c.pads,
                                       c.strides, c.dilations, c.group, c.dtype, relu)
                dc.name = f"DequantizeConv.{dq.name}+{c.name}"
                replace[c.name] = dc
                self.fused_runs.append([dq.name, c.name])
            drop.add(dq.name)
        out_ops = [replace.get(o.name, o) for o in ops if o.name not in drop]
        self.ops = OrderedDict((o.name, o) for o in out_ops)

    def _fuse_runs(self, shapes, consumers):
        ops = list(self.ops.values())
        out_ops = []
        i = 0
        while i < len(ops):
            run = self._run_from(ops, i, shapes, consumers)
            if run is None:
                out_ops.append(ops[i])
                i += 1
                continue
            n_ops, x_in, operands, steps, y_out = run
            chain = Op.ElementwiseChain([x_in] + operands, [y_out], steps, dtype="float32")
            chain.name = "ElementwiseChain." + "+".join(op.name for op in ops[i:i + n_ops])
            self.fused_runs.append([op.name for op in ops[i:i + n_ops]])
            out_ops.append(chain)
            i += n_ops
        self.ops = OrderedDict((op.name, op) for op in out_ops)

    @staticmethod
    def _run_from(ops, i, shapes, consumers):
        """A fusable run starting at ops[i] of at least two nodes, or None."""
        def f32(edge):
            return edge in shapes and shapes[edge][1] == "float32"

        def fits(edge, shape):   # operand broadcasts into the running shape without growing it
            try:
                return np.broadcast_shapes(shapes[edge][0], shape) == tuple(shape)
            except ValueError:
                return False

        steps, operands = [], []
        x_in, cur, shape = None, None, None
        j = i
        while j < len(ops) and len(steps) < 16:
            op = ops[j]
            if not _is_fusable(op) or op.dtype != "float32" or len(op.outputs) != 1 or not f32(op.outputs[0]):
                break
            out = op.outputs[0]
            if cur is None:
                # the running input is one with the output's shape
                cand = [k for k, e in enumerate(op.inputs) if f32(e) and shapes[e][0] == shapes[out][0]]
                if not cand:
                    break
                pos = cand[0]
                x_in, shape = op.inputs[pos], shapes[out][0]
            else:
                if cur not in op.inputs or consumers.get(cur, 0) != 1 or shapes[out][0] != shape:
                    break
                pos = op.inputs.index(cur)
            if type(op) in _UNARY:
                steps.append((_UNARY[type(op)], None, False))
            else:
                other = op.inputs[1 - pos]
                if other == cur or not f32(other) or not fits(other, shape):
                    break
                if other not in operands:
                    if len(operands) == 3:
                        break
                    operands.append(other)
                steps.append((_BINARY[type(op)], operands.index(other), pos == 1))
            cur = out
            j += 1
        if len(steps) < 2:
            return None
        return j - i, x_in, operands, steps, cur
