;;;; hip-vision.lisp -- Qwen3-VL's vision tower on an AMD MI355X through libexn-hip.so
;;;;
;;;; load-vision, vision-encode and vision-release of src/cuda-vision.lisp (:15, :34, :103) with the
;;;; same lambda lists; listed beside hip-dit in ex-nihilo.asd in place of cuda-vision.  Loads after
;;;; hip-dit.lisp, whose shared object, status check and %exn-open it uses.  vision-encode returns
;;;; the merged rows and the three deepstack sets as host vectors (the reference returns device
;;;; buffers of the CUDA prompt encoder's card).

(in-package #:ex-nihilo)

(sb-alien:define-alien-routine ("exn_vision_create" %exn-vision-create) sb-alien:int
  (ctx sb-sys:system-area-pointer) (out sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_vision_set" %exn-vision-set) sb-alien:int
  (v sb-sys:system-area-pointer) (name sb-alien:c-string) (kind sb-alien:int)
  (data sb-sys:system-area-pointer) (dims sb-sys:system-area-pointer) (ndims sb-alien:int))
(sb-alien:define-alien-routine ("exn_vision_check" %exn-vision-check) sb-alien:int (v sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_vision_encode" %exn-vision-encode) sb-alien:int
  (v sb-sys:system-area-pointer) (px sb-sys:system-area-pointer) (h sb-alien:int) (w sb-alien:int)
  (merged sb-sys:system-area-pointer) (deepstack sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_vision_release" %exn-vision-release) sb-alien:int (v sb-sys:system-area-pointer))

(defun load-vision (path &key (device 1))
  "The vision tower in the mmproj GGUF at PATH on HIP device DEVICE: every tensor as floats
   (il::load-f32, as vision-tensors reads them), its shape the GGUF dims reversed (row-major)."
  (let* ((g (read-gguf path))
         (ctx (exn-out-pointer #'%exn-open device))
         (v (exn-out-pointer #'%exn-vision-create ctx)))
    (check-vision g path)
    (dolist (name (gguf-tensor-order g))
      (let* ((f (il::load-f32 g name))
             (shape (reverse (tensor-info-dims (gguf-tensor g name))))
             (dims (make-array (length shape) :element-type '(signed-byte 64) :initial-contents shape)))
        (sb-sys:with-pinned-objects (f dims)
          (exn-check (%exn-vision-set v name +exn-f32+ (sb-sys:vector-sap f) (sb-sys:vector-sap dims)
                                      (length shape))))))
    (exn-check (%exn-vision-check v))
    v))

(defun vision-encode (v px h w)
  "cuda-vision.lisp's vision-encode on the MI355X: PX (H x W RGBA floats, -1 .. 1; H, W
   multiples of 32) through the tower: (values merged deepstack m), MERGED the M x 4096 rows
   (M = H W / 1024, the 32 px grid row-major), DEEPSTACK a list of three more."
  (assert (and (zerop (mod h 32)) (zerop (mod w 32))))
  (let* ((m (* (floor h 32) (floor w 32)))
         (merged (f32vec (* m 4096)))
         (deep (f32vec (* 3 m 4096))))
    (sb-sys:with-pinned-objects (px merged deep)
      (exn-check (%exn-vision-encode v (sb-sys:vector-sap px) h w (sb-sys:vector-sap merged) (sb-sys:vector-sap deep))))
    (values merged
            (loop for j below 3 collect (subseq deep (* j m 4096) (* (1+ j) m 4096)))
            m)))

(defun vision-release (v)
  "V's scratch freed (the weights stay)."
  (exn-check (%exn-vision-release v)))
