;;;; hip-encoder.lisp -- the prompt encoder's text model on an AMD MI355X through libexn-hip.so
;;;;
;;;; load-encoder, encode-prompt and encoder-states of src/encoder.lisp (:41, :55, :143) with the
;;;; reference's lambda lists, for a GPU encoder: the text model's forward runs in libexn-hip.so
;;;; (exn_enc_*) in place of illatio's il::cuda-forward-n; tokenizing stays illatio's
;;;; (il::tokenize on the GGUF's vocabulary).  An edit prompt's picture rows go to the forward as
;;;; arguments instead of through il::*after-embed* / il::*after-layer* (call-with-picture-rows,
;;;; :69-110).  Loads after hip-dit.lisp and hip-vision.lisp, whose shared object, status check,
;;;; %exn-open and vision-encode it uses; listed in ex-nihilo.asd after them.

(in-package #:ex-nihilo)

(sb-alien:define-alien-routine ("exn_enc_create" %exn-enc-create) sb-alien:int
  (ctx sb-sys:system-area-pointer) (layers sb-alien:int) (rope-base sb-alien:double) (out sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_enc_set" %exn-enc-set) sb-alien:int
  (e sb-sys:system-area-pointer) (name sb-alien:c-string) (kind sb-alien:int)
  (data sb-sys:system-area-pointer) (d0 (sb-alien:signed 64)) (d1 (sb-alien:signed 64)))
(sb-alien:define-alien-routine ("exn_enc_check" %exn-enc-check) sb-alien:int (e sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_enc_states" %exn-enc-states) sb-alien:int
  (e sb-sys:system-area-pointer) (ids sb-sys:system-area-pointer) (n sb-alien:int) (pos sb-sys:system-area-pointer)
  (pic0 sb-alien:int) (m sb-alien:int) (merged sb-sys:system-area-pointer) (deep sb-sys:system-area-pointer)
  (out sb-sys:system-area-pointer))
(sb-alien:define-alien-routine ("exn_enc_release" %exn-enc-release) sb-alien:int (e sb-sys:system-area-pointer))

(defstruct (hencoder (:constructor %make-hencoder)) handle tokenizer)

(defun load-encoder (path &key device (threads (il::default-thread-count)))
  "The prompt encoder in the qwen3vl GGUF at PATH: its text model on HIP device DEVICE (0 when
   NIL), every block's matrices as the file's Q8_0 records, its norms as floats; the
   vocabulary through illatio for il::tokenize."
  (let* ((g (read-gguf path)) (file (il::map-file-vector path))
         (ctx (exn-out-pointer #'%exn-open (or device 0)))
         (e (exn-out-pointer #'%exn-enc-create ctx 36 (coerce (meta g "qwen3vl.rope.freq_base") 'double-float))))
    (dolist (name (gguf-tensor-order g))
      (let* ((ti (gguf-tensor g name)) (dims (tensor-info-dims ti)))
        (if (or (null (rest dims)) (eq (tensor-info-type ti) :f32))
            (let ((v (il::load-f32 g name)))
              (sb-sys:with-pinned-objects (v)
                (exn-check (%exn-enc-set e name +exn-f32+ (sb-sys:vector-sap v) (first dims) (reduce #'* (rest dims))))))
            (sb-sys:with-pinned-objects (file)
              (exn-check (%exn-enc-set e name (ecase (tensor-info-type ti) (:q8_0 +exn-q8-0+))
                                       (sb-sys:sap+ (sb-sys:vector-sap file)
                                                    (+ (il::gguf-data-offset g) (il::tensor-info-offset ti)))
                                       (first dims) (reduce #'* (rest dims))))))))
    (exn-check (%exn-enc-check e))
    (%make-hencoder :handle e :tokenizer (il::load-model path :threads threads))))

(defun encoder-states (model ids &key positions picture)
  "Every token's state after the text model's last block, before its final norm: (length IDS)
   x 4096 floats.  POSITIONS: a (t h w) list a token (text positions 0 .. when NIL); PICTURE:
   (a0 merged deep m), the vision tower's rows for tokens a0 .. a0 + m - 1."
  (let* ((n (length ids))
         (iv (make-array n :element-type '(signed-byte 32) :initial-contents (coerce ids 'list)))
         (pv (and positions (make-array (* 3 n) :element-type '(signed-byte 32)
                                                :initial-contents (apply #'append positions))))
         (out (f32vec (* n 4096)))
         (merged (and picture (second picture)))
         (deep (and picture (apply #'concatenate '(simple-array single-float (*)) (third picture)))))
    (sb-sys:with-pinned-objects (iv pv out merged deep)
      (exn-check (%exn-enc-states (hencoder-handle model) (sb-sys:vector-sap iv) n
                                  (if pv (sb-sys:vector-sap pv) (sb-sys:int-sap 0))
                                  (if picture (first picture) 0) (if picture (fourth picture) 0)
                                  (if merged (sb-sys:vector-sap merged) (sb-sys:int-sap 0))
                                  (if deep (sb-sys:vector-sap deep) (sb-sys:int-sap 0))
                                  (sb-sys:vector-sap out))))
    out))

(defun encode-prompt (model prompt &key vision picture)
  "encoder.lisp's encode-prompt with the text model on the MI355X: (values states p a)."
  (let* ((tk (hencoder-tokenizer model))
         (skip (length (il::tokenize tk +system-turn+ :add-bos nil))))
    (if (null picture)
        (let* ((ids (il::tokenize tk (prompt-text prompt) :add-bos nil)) (n (length ids)))
          (values (subseq (encoder-states model ids) (* skip 4096)) (- n skip) 0))
        (destructuring-bind (px h w) picture
          (multiple-value-bind (before after) (edit-prompt-pieces prompt)
            (let* ((b (il::tokenize tk before :add-bos nil)) (e (il::tokenize tk after :add-bos nil))
                   (gh (floor h 32)) (gw (floor w 32)) (m (* gh gw)) (a0 (length b))
                   (ids (concatenate 'vector b (make-array m :initial-element +image-pad+) e))
                   (n (length ids))
                   (positions (append (loop for i below a0 collect (list i i i))
                                      (loop for r below gh
                                            append (loop for c below gw collect (list a0 (+ a0 r) (+ a0 c))))
                                      (loop with p0 = (+ a0 (max gh gw)) for i below (length e)
                                            collect (list (+ p0 i) (+ p0 i) (+ p0 i))))))
              (multiple-value-bind (merged deep) (vision-encode vision px h w)
                (let ((all (encoder-states model ids :positions positions :picture (list a0 merged deep m)))
                      (out (f32vec (* (- n skip m) 4096))))
                  ;; the text's states, the system turn and the picture's rows left out
                  (replace out all :start2 (* skip 4096) :end2 (* a0 4096))
                  (replace out all :start1 (* (- a0 skip) 4096) :start2 (* (+ a0 m) 4096))
                  (vision-release vision)
                  (values out (- n skip m) (- a0 skip))))))))))

(defun encoder-release (model)
  "MODEL's scratch freed (the weights stay)."
  (exn-check (%exn-enc-release (hencoder-handle model))))
