//go:build hip

// The MI355X (gfx950) forward behind futon's native API: built only with
// `go build -tags hip`, which also needs cgo and libfuton_hip.so (the C ABI
// in include/futon_hip.h).  The default pure-Go build never sees this file.
package native

/*
#cgo CFLAGS: -I${SRCDIR}/../third_party/futon_amd/include
#cgo LDFLAGS: -L${SRCDIR}/../third_party/futon_amd -lfuton_hip -Wl,-rpath,${SRCDIR}/../third_party/futon_amd
#include <stdlib.h>
#include "futon_hip.h"
*/
import "C"

import (
	"context"
	"fmt"
	"os"
	"runtime"
	"sync/atomic"
	"unsafe"
)

func init() { accelNew = newHIPModel }

type hipModel struct {
	h   *C.fh_model
	cfg *PackConfig
}

func hipErr(rc C.int) error {
	buf := make([]byte, 1024)
	C.fh_last_error((*C.char)(unsafe.Pointer(&buf[0])), C.size_t(len(buf)))
	return fmt.Errorf("native: hip: %s: %s", C.GoString(C.fh_strerror(rc)), C.GoString((*C.char)(unsafe.Pointer(&buf[0]))))
}

// newHIPModel uploads a pack newModel (model.go:134-295) has validated.  The
// device repeats newModel's tensor-set and shape checks; FUTON_NATIVE_Q8=1
// selects int8 layer weights as the CPU path does (quant.go:30).
func newHIPModel(cfg *PackConfig, tensors map[string]*Tensor) (accelModel, error) {
	var c C.fh_config
	c.hidden_size = C.int32_t(cfg.HiddenSize)
	c.num_layers = C.int32_t(cfg.NumLayers)
	c.num_heads = C.int32_t(cfg.NumHeads)
	c.intermediate_size = C.int32_t(cfg.IntermediateSize)
	c.vocab_size = C.int32_t(cfg.VocabSize)
	c.type_vocab_size = C.int32_t(cfg.TypeVocabSize)
	c.max_seq_len = C.int32_t(cfg.MaxSeqLen)
	c.max_trained_positions = C.int32_t(cfg.MaxTrainedPositions)
	c.layer_norm_eps = C.double(cfg.LayerNormEps)
	if cfg.PositionEncoding == "rope" {
		c.position_encoding = C.FH_POS_ROPE
	}
	c.rope_theta = C.double(cfg.RoPETheta)
	if cfg.Activation == "swiglu" {
		c.activation = C.FH_ACT_SWIGLU
	}
	if cfg.Pooling == "cls" {
		c.pooling = C.FH_POOL_CLS
	}
	if cfg.Normalize {
		c.normalize = 1
	}
	if cfg.Matryoshka != nil {
		c.matryoshka = 1
		if cfg.Matryoshka.LayerNorm {
			c.matryoshka_layernorm = 1
		}
	}
	if os.Getenv("FUTON_NATIVE_Q8") == "1" {
		c.q8 = 1
	}
	// cgo may not pass Go memory holding Go pointers: names and data are
	// copied to C memory for the duration of the call (the library copies
	// them to the device and keeps nothing).
	n := len(tensors)
	ts := unsafe.Slice((*C.fh_tensor)(C.calloc(C.size_t(n), C.size_t(unsafe.Sizeof(C.fh_tensor{})))), n)
	var frees []unsafe.Pointer
	defer func() {
		for _, p := range frees {
			C.free(p)
		}
		C.free(unsafe.Pointer(&ts[0]))
	}()
	i := 0
	for name, t := range tensors {
		if len(t.Shape) > 4 {
			return nil, fmt.Errorf("native: tensor %q has rank %d", name, len(t.Shape))
		}
		cn := C.CString(name)
		frees = append(frees, unsafe.Pointer(cn))
		ts[i].name = cn
		ts[i].rank = C.int32_t(len(t.Shape))
		for d, s := range t.Shape {
			ts[i].shape[d] = C.int64_t(s)
		}
		var p unsafe.Pointer
		if t.F16 != nil {
			ts[i].dtype = C.FH_DTYPE_F16
			p = C.CBytes(unsafe.Slice((*byte)(unsafe.Pointer(unsafe.SliceData(t.F16))), 2*len(t.F16)))
		} else {
			ts[i].dtype = C.FH_DTYPE_F32
			p = C.CBytes(unsafe.Slice((*byte)(unsafe.Pointer(unsafe.SliceData(t.Data))), 4*len(t.Data)))
		}
		frees = append(frees, p)
		ts[i].data = p
		i++
	}
	m := &hipModel{cfg: cfg}
	switch rc := C.fh_model_create(&c, &ts[0], C.int32_t(n), 0, &m.h); rc {
	case C.FH_OK:
	case C.FH_ENODEV:
		return nil, nil // no gfx950 device: keep the CPU path
	default:
		return nil, hipErr(rc)
	}
	runtime.SetFinalizer(m, func(m *hipModel) { m.Close() })
	return m, nil
}

// EncodeBatch runs EncodeTokensKernel (model.go:346-457) for every sequence
// in one device call.  ctx is watched by a goroutine that raises the flag
// the device forward polls between layers as they execute.
func (m *hipModel) EncodeBatch(ctx context.Context, batch [][]int, outDim int) ([][]float32, error) {
	if len(batch) == 0 {
		return nil, nil
	}
	total := 0
	for _, ids := range batch {
		total += len(ids)
	}
	dim := outDim
	if dim == 0 {
		dim = m.cfg.HiddenSize
	}
	if dim < 1 || dim > m.cfg.HiddenSize {
		return nil, fmt.Errorf("native: requested dim %d outside [1,%d]", outDim, m.cfg.HiddenSize)
	}
	ids := unsafe.Slice((*C.int32_t)(C.malloc(C.size_t(4*(total+1)))), total+1)
	offs := unsafe.Slice((*C.int32_t)(C.malloc(C.size_t(4*(len(batch)+1)))), len(batch)+1)
	out := unsafe.Slice((*C.float)(C.malloc(C.size_t(4*len(batch)*dim))), len(batch)*dim)
	cancel := (*C.int32_t)(C.malloc(4))
	defer func() {
		C.free(unsafe.Pointer(&ids[0]))
		C.free(unsafe.Pointer(&offs[0]))
		C.free(unsafe.Pointer(&out[0]))
		C.free(unsafe.Pointer(cancel))
	}()
	k := 0
	for i, seq := range batch {
		offs[i] = C.int32_t(k)
		for _, id := range seq {
			if id < -1<<31 || id > 1<<31-1 {
				return nil, fmt.Errorf("native: batch item %d: native: token id %d outside vocab of %d", i, id, m.cfg.VocabSize)
			}
			ids[k] = C.int32_t(id)
			k++
		}
	}
	offs[len(batch)] = C.int32_t(k)
	*cancel = 0
	done := make(chan struct{})
	defer close(done)
	go func() {
		select {
		case <-ctx.Done():
			atomic.StoreInt32((*int32)(unsafe.Pointer(cancel)), 1)
		case <-done:
		}
	}()
	rc := C.fh_encode(m.h, &ids[0], &offs[0], C.int32_t(len(batch)), C.int32_t(outDim), &out[0], cancel)
	if rc == C.FH_ECANCELED {
		return nil, ctx.Err() // nil vectors, as TestCancellationInsideLayer requires
	}
	if rc != C.FH_OK {
		return nil, hipErr(rc)
	}
	res := make([][]float32, len(batch))
	for i := range res {
		res[i] = make([]float32, dim)
		for j := range res[i] {
			res[i][j] = float32(out[i*dim+j])
		}
	}
	return res, nil
}

func (m *hipModel) Close() error {
	if m.h != nil {
		C.fh_model_destroy(m.h)
		m.h = nil
	}
	return nil
}
