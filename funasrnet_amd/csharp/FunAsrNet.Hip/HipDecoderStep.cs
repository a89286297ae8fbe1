using System.Runtime.InteropServices;

namespace FunAsrNet.Hip;

/// <summary>QwenDecoder on the device (fah_decoder_*): built from the Qwen3 GGUF's
/// Q8_0 tensors, keeps its F16 K/V cache, position and the last logits' greedy
/// token on the device.</summary>
public sealed unsafe class HipDecoderStep : IDecoderStep
{
    private IntPtr _decoder;
    private readonly HipStepBatcher? _batcher;
    private bool _joined;   // registered with the batcher: this decoder is stepping

    private HipDecoderStep(IntPtr decoder, HipStepBatcher? batcher)
    {
        _decoder = decoder;
        _batcher = batcher;
        _batcher?.AddUser();
    }

    /// <summary>True once <see cref="Dispose"/> has run.</summary>
    internal bool IsDisposed => _decoder == IntPtr.Zero;

    internal IntPtr Handle
    {
        get
        {
            ObjectDisposedException.ThrowIf(_decoder == IntPtr.Zero, this);
            return _decoder;
        }
    }

    /// <summary>The shapes fah_decoder_create takes (funasr_hip.h): head size 128,
    /// 2 or 4 query heads per KV head, widths multiples of 32 with the model and
    /// q widths at most 4096 and the ffn width at most 16384 (Qwen3-0.6B to 8B).</summary>
    internal static bool ShapeSupported(in Native.DecoderConfig c) =>
        c.HeadSize == 128 && c.KvHeads > 0 && (c.Heads == 2 * c.KvHeads || c.Heads == 4 * c.KvHeads) &&
        c.Width % 32 == 0 && c.Ffn % 32 == 0 && c.Width <= 4096 && c.Heads * c.HeadSize <= 4096 && c.Ffn <= 16384;

    /// <summary>fah_decoder_create from the model's tensors (names and metadata of
    /// QwenDecoder.cs:46-75); null when the shape is not one the library takes
    /// (the reference's own decoder then runs) or a tensor is not Q8_0 in
    /// row-major form. Step batching needs an ffn width of at most 3072; larger
    /// models step on their own.</summary>
    internal static HipDecoderStep? Create(IntPtr context, Gguf model, int capacity, bool batching)
    {
        int layers = model.Int("qwen3.block_count", 28);
        var embd = model["token_embd.weight"];
        model.Tensors.TryGetValue("output.weight", out var output);
        var config = new Native.DecoderConfig
        {
            Width = model.Int("qwen3.embedding_length", 1024),
            Heads = model.Int("qwen3.attention.head_count", 16),
            KvHeads = model.Int("qwen3.attention.head_count_kv", 8),
            HeadSize = model.Int("qwen3.attention.key_length", 128),
            Layers = layers,
            Ffn = model["blk.0.ffn_gate.weight"].Rows,
            Vocab = embd.Rows,
            Eps = model.Float("qwen3.attention.layer_norm_rms_epsilon", 1e-6f),
            RopeBase = model.Float("qwen3.rope.freq_base", 1000000),
            Capacity = capacity,
        };
        if (!ShapeSupported(config))
        {
            return null;
        }
        batching &= config.Ffn <= 3072;
        var pins = new List<GCHandle>();
        try
        {
            float* Pin(float[] a)
            {
                var h = GCHandle.Alloc(a, GCHandleType.Pinned);
                pins.Add(h);
                return (float*)h.AddrOfPinnedObject();
            }
            bool Q8(Weight w, out Native.Q8Host host)
            {
                host = default;
                if (w.Quantized is null || w.Scales is null || w.QuantizedInterleaved)
                {
                    return false;
                }
                var q = GCHandle.Alloc(w.Quantized, GCHandleType.Pinned);
                pins.Add(q);
                host.Quantized = (sbyte*)q.AddrOfPinnedObject();
                host.Scales = Pin(w.Scales);
                host.Rows = w.Rows;
                host.Cols = w.Columns;
                return true;
            }
            var hostLayers = new Native.LayerHost[layers];
            for (int l = 0; l < layers; l++)
            {
                string p = $"blk.{l}.";
                ref var L = ref hostLayers[l];
                if (!Q8(model[p + "attn_q.weight"], out L.Wq) || !Q8(model[p + "attn_k.weight"], out L.Wk)
                    || !Q8(model[p + "attn_v.weight"], out L.Wv) || !Q8(model[p + "attn_output.weight"], out L.Wo)
                    || !Q8(model[p + "ffn_gate.weight"], out L.Gate) || !Q8(model[p + "ffn_up.weight"], out L.Up)
                    || !Q8(model[p + "ffn_down.weight"], out L.Down))
                {
                    return null;
                }
                L.AttnNorm = Pin(model[p + "attn_norm.weight"].Values!);
                L.QNorm = Pin(model[p + "attn_q_norm.weight"].Values!);
                L.KNorm = Pin(model[p + "attn_k_norm.weight"].Values!);
                L.FfnNorm = Pin(model[p + "ffn_norm.weight"].Values!);
            }
            if (!Q8(embd, out var embdHost))
            {
                return null;
            }
            Native.Q8Host outputHost = default;
            if (output is not null && !Q8(output, out outputHost))
            {
                return null;
            }
            float* outputNorm = Pin(model["output_norm.weight"].Values!);
            IntPtr decoder;
            fixed (Native.LayerHost* lp = hostLayers)
            {
                Native.Check(Native.fah_decoder_create(context, &config, lp, &embdHost,
                    output is null ? null : &outputHost, outputNorm, out decoder));
            }
            // The host arrays may be released now: the weights live on the device.
            HipStepBatcher? batcher = null;
            if (batching)
            {
                try
                {
                    batcher = new HipStepBatcher(decoder, capacity);
                }
                catch
                {
                    Native.fah_decoder_destroy(decoder);
                    throw;
                }
            }
            return new HipDecoderStep(decoder, batcher);
        }
        finally
        {
            foreach (var h in pins)
            {
                h.Free();
            }
        }
    }

    /// <summary>A decoder over the same device weights with its own K/V
    /// (fah_decoder_create_session), stepped through the same batcher.</summary>
    internal HipDecoderStep CreateSession(int capacity)
    {
        Native.Check(Native.fah_decoder_create_session(Handle, capacity, out var session));
        return new HipDecoderStep(session, _batcher);
    }

    public int Position
    {
        get
        {
            Native.Check(Native.fah_decoder_position(Handle, out int position));
            return position;
        }
    }

    public void SetPosition(int position)
    {
        Leave();
        Native.Check(Native.fah_decoder_set_position(Handle, position));
    }

    public void Decode(float[] embeddings, int frames, float[]? logits)
    {
        if (frames > 1)
        {
            Leave();   // a prefill: the next request's first step joins again
        }
        fixed (float* x = embeddings) fixed (float* y = logits)
        {
            Native.Check(Native.fah_decoder_decode(Handle, x, frames, y));
        }
    }

    /// <summary>Greedy -> Embed -> Decode(1) (FunAsr.cs:167-178). With a batcher the
    /// decoder joins it at its first step after a prefill, so the collecting thread
    /// waits only for decoders that are stepping; a decoder whose next position is
    /// past the batcher's bound steps on its own.</summary>
    public int NextToken()
    {
        if (_batcher is not null && Position < _batcher.MaxPositions)
        {
            if (!_joined)
            {
                _batcher.Join(this);
                _joined = true;
            }
            return _batcher.Step(this);
        }
        int token;
        Native.Check(Native.fah_decoder_generate(Handle, 1, &token));
        return token;
    }

    private void Leave()
    {
        if (_joined)
        {
            _batcher!.Leave(this);
            _joined = false;
        }
    }

    public void Dispose()
    {
        if (_decoder == IntPtr.Zero)
        {
            return;
        }
        Leave();
        IntPtr decoder = _decoder;
        _decoder = IntPtr.Zero;
        Native.Check(Native.fah_decoder_destroy(decoder));
        // The batcher is shared by the first decoder of a model and its
        // sessions; the last of them to go destroys it.
        _batcher?.ReleaseUser();
    }
}
