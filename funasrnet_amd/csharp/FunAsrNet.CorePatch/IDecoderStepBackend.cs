namespace FunAsrNet;

// Added to the core assembly (src/FunAsrNet) next to IAttentionComputeBackend.cs.
// QwenDecoder probes it at its first Decode (QwenDecoder.cs:161), where its
// private model and capacity are in scope; INTEGRATION.md shows the lines.

/// <summary>Optional backend that runs the whole decoder step on a device (norms,
/// projections, QK-norm, RoPE, F16 KV cache, attention, SwiGLU, lm_head, greedy).
/// Once it accepts a decoder, the device owns that decoder's K/V rows.</summary>
public interface IDecoderStepBackend
{
    /// <summary>Builds a device decoder for the Qwen3 GGUF <paramref name="model"/>
    /// with room for <paramref name="capacity"/> positions; false leaves the CPU path.</summary>
    bool TryCreateDecoder(Gguf model, int capacity, out IDecoderStep? step);
}

/// <summary>A device-resident QwenDecoder (the device keeps position, K/V and the
/// last logits' greedy token).</summary>
public interface IDecoderStep : IDisposable
{
    int Position { get; }
    void SetPosition(int position);
    /// <summary>QwenDecoder.Decode: frames rows at the current position; logits of
    /// the last row into <paramref name="logits"/> when it is not null.</summary>
    void Decode(float[] embeddings, int frames, float[]? logits);
    /// <summary>The greedy token of the last decode's logits, then that token
    /// embedded and decoded (Greedy -> Embed -> Decode(1) on the device).</summary>
    int NextToken();
}
