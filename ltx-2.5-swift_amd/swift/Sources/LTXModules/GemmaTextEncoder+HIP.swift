// The `.hip` case of `GemmaTextEncoder.AttentionPath`: one layer's attention
// (GemmaTextEncoder.swift:158-239 -- projections, q/k/v norms, RoPE, the KV-head repeat, the
// masked SDPA of :288-321 and o_proj) with everything from the projections to the merged
// output in one `ltx_gemma_attn_fwd` call on the selected MI355X. The projections and o_proj
// stay MLX matmuls, as in the reference.
//
// Operands travel through the same context as the DiT path (`HIPDiTCore.context()`): one
// page-locked and one device arena, reused from call to call.
//
// Uncompiled here: the build image has no Swift toolchain.

import Foundation
import LTXAttention
import LTXCatalog
import LTXFoundation
import MLX

enum HIPGemmaCore {
    /// The prompt's left padding: the count of leading zero token weights. The tokenizer
    /// pads on the left (TextConditioningPipeline.swift:12, :37) and the kernel's mask takes
    /// padding as a prefix of the keys; any other pattern is refused rather than computed
    /// under a different mask.
    static func leftPadding(_ tokenWeights: [Float]) throws -> Int32 {
        let lead = tokenWeights.prefix { $0 == 0 }.count
        guard tokenWeights.dropFirst(lead).allSatisfy({ $0 != 0 }) else {
            throw HIPAttention.Failure.unsupported(
                "attentionPath .hip: the text encoder's padding must be a prefix of the "
                    + "prompt (left padding)")
        }
        return Int32(lead)
    }

    /// One layer's attention from its input `x` `[1, T, hidden]`: q/k(/v) projections in
    /// MLX, then norms, RoPE, GQA and the masked SDPA in the library, then o_proj in MLX.
    /// `cos` / `sin` are the layer's tables as `attention` receives them, `[1, T, 1, D]`
    /// with duplicated halves; the library takes their first halves as fp32 `[T, D/2]`
    /// (the values the reference multiplies by, in its dtype).
    static func layer(x: MLXArray, wq: MLXArray, wk: MLXArray, wv: MLXArray?,
                      qNorm: MLXArray, kNorm: MLXArray, wo: MLXArray,
                      shape: TextEncoderTopology.AttentionShape, window: Int, eps: Double,
                      cos: MLXArray, sin: MLXArray, leftPadding: Int32) throws -> MLXArray {
        let ctx = try HIPDiTCore.context()
        let T = x.dim(1), D = shape.headDim
        let Hq = shape.queryHeads, Hkv = shape.keyValueHeads
        let half = D / 2
        let q = MLX.matmul(x, wq.transposed(1, 0))                  // [1, T, Hq * D]
        let k = MLX.matmul(x, wk.transposed(1, 0))                  // [1, T, Hkv * D]
        let v = wv.map { MLX.matmul(x, $0.transposed(1, 0)) }       // nil: V from pre-norm K
        let c = cos.reshaped([T, D])[0..., 0 ..< half].asType(.float32)
        let s = sin.reshaped([T, D])[0..., 0 ..< half].asType(.float32)

        var lay = HIPAttentionContext.Layout()
        let nq = T * Hq * D, nk = T * Hkv * D
        let oq = lay.place(2 * nq), ok = lay.place(2 * nk)
        let ov = v == nil ? ok : lay.place(2 * nk)
        let owq = lay.place(2 * D), owk = lay.place(2 * D)
        let oc = lay.place(4 * T * half), os = lay.place(4 * T * half)
        let inputBytes = lay.bytes
        let oout = lay.place(4 * nq)
        let (host, device) = try ctx.arenas(bytes: lay.bytes)
        try HIPDiTCore.stage(q, count: nq, into: host, at: oq)
        try HIPDiTCore.stage(k, count: nk, into: host, at: ok)
        if let v { try HIPDiTCore.stage(v, count: nk, into: host, at: ov) }
        try HIPDiTCore.stage(qNorm, count: D, into: host, at: owq)
        try HIPDiTCore.stage(kNorm, count: D, into: host, at: owk)
        for (table, offset) in [(c, oc), (s, os)] {
            let f = table.flattened().asArray(Float.self)
            guard f.count == T * half else {
                throw HIPAttention.Failure.invalid("rope table of \(f.count) values, expected "
                                                   + "\(T * half)")
            }
            f.withUnsafeBytes { src in
                (host + offset).copyMemory(from: src.baseAddress!, byteCount: src.count)
            }
        }
        try ctx.upload(bytes: inputBytes)

        let call = HIPGemmaAttention.Call(
            batch: 1, tokens: Int32(T), queryHeads: Int32(Hq), keyValueHeads: Int32(Hkv),
            headDim: Int32(D), q: device + oq, k: device + ok, v: device + ov,
            qRowStride: Int64(Hq * D), kRowStride: Int64(Hkv * D), vRowStride: Int64(Hkv * D),
            qNormWeight: device + owq, kNormWeight: device + owk, eps: Float(eps),
            cos: device + oc, sin: device + os, window: Int32(window),
            leftPadding: [leftPadding], scale: GemmaAttentionSpec.attentionScaling,
            out: device + oout)
        let bytes = try HIPGemmaAttention.workspaceBytes(call)
        guard let ws = try ctx.workspace(bytes: bytes) else {
            throw HIPAttention.Failure.invalid("the text-encoder attention needs a workspace")
        }
        try HIPGemmaAttention.attend(call, workspace: ws.pointer, workspaceBytes: bytes,
                                     stream: ctx.stream)
        try ctx.download(offset: oout, bytes: 4 * nq)
        let merged = Array(UnsafeBufferPointer(
            start: (host + oout).assumingMemoryBound(to: Float.self), count: nq))
        // the explicit path's output dtype (`.asType(q.dtype)`, :229), then o_proj (:236-238)
        let out = MLXArray(merged, [1, T, Hq * D]).asType(x.dtype)
        return MLX.matmul(out, wo.transposed(1, 0))
    }
}
