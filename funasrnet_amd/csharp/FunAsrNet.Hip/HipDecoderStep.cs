using System.Runtime.InteropServices;

namespace FunAsrNet.Hip;

/// <summary>QwenDecoder on the device (fah_decoder_*): built from the Qwen3 GGUF's
/// Q8_0 tensors, keeps its F16 K/V cache, position and the last logits' greedy
/// token on the device.</summary>
public sealed unsafe class HipDecoderStep : IDecoderStep
{
    private IntPtr _decoder;
    private readonly HipStepBatcher? _batcher;
    private readonly List<HipDecoderStep> _sessions = [];

    private HipDecoderStep(IntPtr decoder, HipStepBatcher? batcher)
    {
        _decoder = decoder;
        _batcher = batcher;
        _batcher?.Join(this);
    }

    internal IntPtr Handle
    {
        get
        {
            ObjectDisposedException.ThrowIf(_decoder == IntPtr.Zero, this);
            return _decoder;
        }
    }

    /// <summary>fah_decoder_create from the model's tensors (names and metadata of
    /// QwenDecoder.cs:46-75); null when a tensor is not Q8_0 in row-major form.</summary>
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
            var batcher = batching ? new HipStepBatcher(decoder, capacity) : null;
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
        var step = new HipDecoderStep(session, _batcher);
        _sessions.Add(step);
        return step;
    }

    public int Position
    {
        get
        {
            Native.Check(Native.fah_decoder_position(Handle, out int position));
            return position;
        }
    }

    public void SetPosition(int position) => Native.Check(Native.fah_decoder_set_position(Handle, position));

    public void Decode(float[] embeddings, int frames, float[]? logits)
    {
        fixed (float* x = embeddings) fixed (float* y = logits)
        {
            Native.Check(Native.fah_decoder_decode(Handle, x, frames, y));
        }
    }

    public int NextToken()
    {
        if (_batcher is not null)
        {
            return _batcher.Step(this);
        }
        int token;
        Native.Check(Native.fah_decoder_generate(Handle, 1, &token));
        return token;
    }

    public void Dispose()
    {
        if (_decoder == IntPtr.Zero)
        {
            return;
        }
        _batcher?.Leave(this);
        if (_sessions.Count == 0 && _batcher is not null && _batcher.Owner == _decoder)
        {
            _batcher.Dispose();
        }
        Native.fah_decoder_destroy(_decoder);
        _decoder = IntPtr.Zero;
    }
}
